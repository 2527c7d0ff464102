"""GGUF weight residency on the device (include/qw6_gguf.h): MoE layers and
the output head written to GGUF files, made resident by the library's loader
and run through the kernels.

Bars:
 - the same bytes made resident by the loader and by the synthetic-layer
   path give bit-identical outputs and indices (the loader binds exactly the
   expert-pack layout qw6 defines);
 - against the oracle on the bytes written: expert indices bit-exact, rel-L2
   <= 1e-5 (the fp32 kernels' bar), with the shared-expert gate and the
   RMSNorm weight read from the file;
 - the output head's token equals the oracle's argmax.
"""
from __future__ import annotations

import sys
import time

import numpy as np
import pytest

import cases
import oracle as O
import qw6_amd as Q
from qw6_amd import gguf as G
from qw6_amd import synth as S

pytestmark = pytest.mark.gpu

TOL = 1e-5
TIE = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "no GPU visible"
    return torch


@pytest.fixture(scope="module")
def ctx(torch_dev):
    c = Q.Context(0, max_tokens=64)
    yield c
    c.close()


def export_layer(path, L, layer_id, shared_router=None, norm_w=None, kv_extra=()):
    """Write a SynthLayer's bytes as blk.<layer_id> of a GGUF file."""
    packs = []
    for k in range(3):
        qs = {L.quants[e][k] for e in range(L.n_experts)}
        assert len(qs) == 1, "a GGUF expert pack has one type"
        packs.append((qs.pop(), [L.expert_host(e)[k][0] for e in range(L.n_experts)]))
    ts = G.moe_layer_tensors(layer_id, L.hidden, L.inter, L.router_host(), packs,
                             shared=L.shared_host(), shared_router=shared_router, norm_w=norm_w)
    kv = [("general.architecture", G.T_STR, "qwen35moe"),
          ("qwen35moe.expert_count_used", G.T_U32, L.top_k)] + list(kv_extra)
    return G.write_gguf(path, kv, ts)


def run(torch, ctx, desc, xs, hidden, top_k):
    T = xs.shape[0]
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    out = torch.zeros(T, hidden, dtype=torch.float32, device="cuda")
    idx = torch.zeros(T, top_k, dtype=torch.int32, device="cuda")
    ctx.moe_forward(desc, dx, out, n_tok=T, idx=idx)
    torch.cuda.synchronize()
    return out, idx


@pytest.mark.parametrize("mix", ["q4k", "iq2a"])
def test_gguf_layer_equals_resident_layer(torch_dev, ctx, tmp_path, mix):
    """hidden 512, inter 256, 64 experts, top-8 from the file's metadata,
    shared expert with its gate, RMSNorm weight: T = 1, 2, 3, 4, 8, 40 through
    every path (fp32 per-token, small-batch MFMA, grouped), bit-identical
    to the synthetic layer carrying the same gate and norm buffers."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    say("gguf layer vs resident", mix)
    L = SynthLayer(ctx, 71, 0, mix, hidden=512, inter=256, n_experts=64)
    try:
        sr = S.f32_normal(71, S.stream_id(0, S.K_SROUTER), 512, 0.02)
        nw = cases.norm_w(71, 0, hidden=512)
        p = tmp_path / "layer.gguf"
        export_layer(p, L, 5, shared_router=sr, norm_w=nw)
        with G.GgufFile(p) as f:
            desc, E = f.moe_layer(ctx, 5)
        try:
            assert (desc.hidden, desc.inter, desc.top_k) == (512, 256, 8)
            assert desc.shared_router and desc.norm_w and desc.norm_eps == pytest.approx(1e-6)
            ref = Q.MoeLayer.from_buffer_copy(L.desc)
            ref.shared_router, ref.norm_w, ref.norm_eps = desc.shared_router, desc.norm_w, desc.norm_eps
            for T in (1, 2, 3, 4, 8, 40):
                xs = np.stack([cases.token_x(710 + T, 1, t, hidden=512) for t in range(T)])
                o1, i1 = run(torch, ctx, desc, xs, 512, 8)
                o2, i2 = run(torch, ctx, ref, xs, 512, 8)
                assert torch.equal(i1, i2), T
                assert torch.equal(o1, o2), T
        finally:
            E.free()
    finally:
        L.free()


@pytest.mark.parametrize("mix", ["q4k", "iq2b"])
def test_gguf_layer_vs_oracle(torch_dev, ctx, tmp_path, mix):
    """The loaded layer against the oracle on the written bytes: RMSNorm
    with the file's weight and epsilon, the shared expert weighted by
    sigmoid(shared_router . x), top-6 from the file's metadata."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    say("gguf layer vs oracle", mix)
    H, I, N, K = 512, 256, 32, 6
    L = SynthLayer(ctx, 72, 0, mix, hidden=H, inter=I, n_experts=N, top_k=K)
    try:
        sr = S.f32_normal(72, S.stream_id(0, S.K_SROUTER), H, 0.02)
        nw = cases.norm_w(72, 0, hidden=H)
        eps = 1e-5
        p = tmp_path / "layer.gguf"
        export_layer(p, L, 0, shared_router=sr, norm_w=nw,
                     kv_extra=[("qwen35moe.attention.layer_norm_rms_epsilon", G.T_F32, eps)])
        router = L.router_host()
        ol = O.Layer(H, I, N, K, router, [L.expert_host(e) for e in range(N)], L.shared_host(), sr)
        with G.GgufFile(p) as f:
            desc, E = f.moe_layer(ctx, 0)
        try:
            assert desc.top_k == K and desc.norm_eps == pytest.approx(eps)
            n = 0
            for T in (1, 3):
                xs = np.stack([cases.token_x(720 + T, 1, t, hidden=H) for t in range(T)])
                out, idx = run(torch, ctx, desc, xs, H, K)
                out, idx = out.cpu().numpy(), idx.cpu().numpy()
                for t in range(T):
                    xn = O.rmsnorm(xs[t], nw, eps)
                    want, widx, _ = O.moe_layer(ol, xn)
                    if cases.route_gap(O.matvec(0, router, N, H, xn), K) < TIE:
                        say("near tie skipped", T, t)
                        continue
                    assert np.array_equal(idx[t], widx), (T, t)
                    assert cases.rel_l2(out[t], want) <= TOL, (T, t)
                    n += 1
            assert n >= 3
        finally:
            E.free()
    finally:
        L.free()


def test_gguf_full_size_layer(torch_dev, ctx, tmp_path):
    """hidden 2048, inter 512, 256 Q4_K / Q6_K experts: 151 / 151 / 220 MB
    packs streamed through the 32 MiB staging buffers; bit-identical to the
    synthetic layer at 1 and 4 tokens."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 73, 0, "q4k")
    try:
        p = tmp_path / "big.gguf"
        export_layer(p, L, 39)
        size = p.stat().st_size
        with G.GgufFile(p) as f:
            t0 = time.perf_counter()
            desc, E = f.moe_layer(ctx, 39)
            dt = time.perf_counter() - t0
        say("loaded %.1f MB in %.3f s (%.2f GB/s file -> HBM)" % (size / 1e6, dt, size / dt / 1e9))
        try:
            for T in (1, 4):
                xs = np.stack([cases.token_x(730 + T, 1, t) for t in range(T)])
                o1, i1 = run(torch, ctx, desc, xs, 2048, 8)
                o2, i2 = run(torch, ctx, L.desc, xs, 2048, 8)
                assert torch.equal(i1, i2) and torch.equal(o1, o2), T
        finally:
            E.free()
    finally:
        L.free()


def test_gguf_output_head(torch_dev, ctx, tmp_path):
    """output.weight (Q6_K [2048, 5000]) and output_norm.weight uploaded
    from the file; the greedy head's token equals the oracle's argmax of the
    oracle's logits, which agree to rel-L2 1e-5."""
    torch = torch_dev
    H, V = 2048, 5000
    w = S.quant_matrix(74, S.stream_id(0, S.K_OUTPUT), S.Q_Q6_K, V, H)
    nw = S.f32_normal(74, S.stream_id(0, S.K_ONORM), H, 0.1, mean=1.0)
    p = tmp_path / "head.gguf"
    G.write_gguf(p, [("general.architecture", G.T_STR, "qwen35moe")],
                 [("output_norm.weight", G.G_F32, [H], nw), ("output.weight", G.G_Q6_K, [H, V], w)])
    with G.GgufFile(p) as f:
        wm = f.upload(ctx, f.find("output.weight"))
        nm = f.upload(ctx, f.find("output_norm.weight"))
    assert wm[1:] == (S.Q_Q6_K, V, H) and nm[1:] == (0, 1, H)
    x = cases.token_x(74, 0)
    dx = torch.from_numpy(x).cuda()
    logits = torch.zeros(V, dtype=torch.float32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.output_greedy(wm, dx, logits, tok, norm_w=nm[0])
    torch.cuda.synchronize()
    want = O.matvec(S.Q_Q6_K, w, V, H, O.rmsnorm(x, nw))
    assert cases.rel_l2(logits.cpu().numpy(), want) <= TOL
    s = np.sort(want)[::-1]
    assert s[0] - s[1] > 1e-3
    assert int(tok.cpu()[0]) == O.argmax(want)


def test_gguf_layer_errors(torch_dev, ctx, tmp_path):
    """Missing tensors are named; a non-F32 router, packs of another expert
    count, and a partial shared expert are refused before any upload."""
    H, I, N = 256, 256, 8
    router = np.zeros(N * H, np.float32)
    q4 = [np.zeros(S.row_bytes(S.Q_Q4_K_M, H) * I, np.uint8)] * N
    q6 = [np.zeros(S.row_bytes(S.Q_Q6_K, I) * H, np.uint8)] * N
    packs = [(S.Q_Q4_K_M, q4), (S.Q_Q4_K_M, q4), (S.Q_Q6_K, q6)]
    full = G.moe_layer_tensors(0, H, I, router, packs,
                               shared=[(q4[0][:S.row_bytes(S.Q_Q4_K_M, H) * I], S.Q_Q4_K_M)] * 2 +
                               [(q6[0], S.Q_Q6_K)])

    def attempt(tensors, match, layer=0):
        p = tmp_path / "bad.gguf"
        G.write_gguf(p, [], tensors)
        with G.GgufFile(p) as f:
            with pytest.raises(Q.Qw6HipError, match=match):
                f.moe_layer(ctx, layer)

    attempt(full, "layer 3 is missing required tensors: ffn_gate_inp.weight ffn_gate_exps", layer=3)
    attempt([t for t in full if "up_exps" not in t[0]], "missing required tensors: ffn_up_exps")
    attempt([t for t in full if "down_shexp" not in t[0]], "missing required tensors: ffn_down_shexp")
    bad_router = [("blk.0.ffn_gate_inp.weight", G.G_F16, [H, N], np.zeros(N * H, np.uint16))] + full[1:]
    attempt(bad_router, "F32")
    wide = [("blk.0.ffn_gate_inp.weight", G.G_F32, [H, 2 * N], np.zeros(2 * N * H, np.float32))]
    attempt(wide + full[1:], r"is not \[cols, rows, 16\]: 3 dims, the last 8")
