"""Parity of the HIP path with the oracle (and through it, with qw6's own CPU
path via the golden fixtures), called through the C ABI.

Bars: expert indices bit-exact; fp32 outputs rel-L2 <= 1e-5 against the
oracle. Layer/stack routing is compared exactly unless the 8th/9th router
logit gap is below 1e-4 (near tie: GPU and CPU sum the router dot product in
different orders), which is reported and must stay rare.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import cases
import oracle as O
import qw6_amd as Q
from qw6_amd import synth as S

pytestmark = pytest.mark.gpu

G = np.load(Path(__file__).parent / "golden" / "golden.npz")
FORMATS = [S.Q_Q4_K_M, S.Q_Q5_K, S.Q_Q6_K, S.Q_IQ2_XXS, S.Q_IQ2_S, S.Q_IQ3_S]
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
    c = Q.Context(0, max_tokens=4)
    yield c
    c.close()


# ---- host operations -----------------------------------------------------------

@pytest.mark.parametrize("q", FORMATS)
@pytest.mark.parametrize("shape", [(3, 256), (16, 512), (8, 2048), (5, 1280), (130, 2048),
                                   (37, 512), (70, 1024), (9, 4096)])
def test_host_matmul_vs_oracle(q, shape):
    rows, cols = shape
    say("matmul_host q=%d %dx%d" % (q, rows, cols))
    w = S.quant_matrix(3, S.stream_id(0, S.K_GATE, q), q, rows, cols)
    x = S.f32_normal(3, S.stream_id(0, S.K_X, q), cols, 1.0)
    y = Q.matmul_host(q, w, x, rows, cols)
    want = O.matvec(q, w, rows, cols, x)
    assert cases.rel_l2(y, want) <= TOL


def test_host_cfg0_vs_golden():
    w = S.quant_matrix(1, S.stream_id(0, S.K_GATE), S.Q_Q4_K_M, 512, 2048)
    x = S.f32_normal(1, S.stream_id(0, S.K_X), 2048, 1.0)
    y = Q.matmul_host(S.Q_Q4_K_M, w, x, 512, 2048)
    assert cases.rel_l2(y, G["cfg0_y"]) <= TOL


def test_fp16_scales_exhaustive_through_q4k_kernel():
    """Every binary16 d value (subnormals, +-0, inf, NaN) decoded by the
    kernel equals IEEE binary16 -> binary32: one Q4_K block per row with
    sc0 = 1, q0 = 1, x = e_0, so y[r] = d(r)."""
    rows = 65536
    w = np.zeros((rows, 144), np.uint8)
    h = np.arange(rows, dtype=np.uint32)
    w[:, 0] = h & 0xFF
    w[:, 1] = h >> 8
    w[:, 4] = 1          # sub-block 0 scale 1, min 0
    w[:, 16] = 1         # q[0] = 1
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    y = Q.matmul_host(S.Q_Q4_K_M, w.reshape(-1), x, rows, 256)
    d = h.astype(np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(d)
    assert np.array_equal(y[fin], d[fin])
    # inf / NaN d: qw6 multiplies d by the zero scales of the other sub-blocks,
    # so the row is NaN there too; the oracle agrees on every row
    want = O.matvec(S.Q_Q4_K_M, w.reshape(-1), rows, 256, x)
    assert np.array_equal(np.isnan(y), np.isnan(want))
    assert np.array_equal(y[~np.isnan(y)], want[~np.isnan(want)])


def test_host_f32_matvec_kat():
    rows, cols = 7, 19   # qw6_vk.c:1585-1607
    r_, c_ = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    w = (np.float32(0.01) * (r_ - c_)).astype(np.float32)
    x = np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.2)).astype(np.float32)
    y = Q.matmul_host(Q.Q_FP32, w, x, rows, cols)
    assert np.abs(y - O.matvec(0, w.reshape(-1), rows, cols, x)).max() < 2e-5


@pytest.mark.parametrize("name", ["route_randn", "route_ties", "route_small", "route_vkkat",
                                  "route_neginf", "route_n7k3", "route_allequal"])
def test_host_route_exact(name):
    lg, k = cases.route_cases()[name]
    idx, w = Q.moe_route_host(lg, k)
    assert np.array_equal(idx.astype(np.int32), G[name + "_idx"])
    assert np.abs(w - G[name + "_w"]).max() <= 2e-5


def test_host_route_nan_logits_vs_oracle():
    """NaN router logits: the device routing gives qw6's indices (a NaN at
    index 0 selected first, NaNs elsewhere never) and weights (all NaN when
    the first pick is a NaN), against the oracle; plus 256-expert vectors with
    NaNs scattered, at index 0 and not."""
    rng = np.random.default_rng(17)
    vecs = [(np.array(lg, np.float32), k) for lg, k, _ in cases.nan_route_cases()]
    for trial in range(12):
        lg = rng.standard_normal(256).astype(np.float32)
        lg[rng.integers(0, 256, 1 + trial)] = np.nan
        if trial % 3 == 0:
            lg[0] = np.nan
        vecs.append((lg, 8))
    for lg, k in vecs:
        idx, w = Q.moe_route_host(lg, k)
        oi, ow = O.moe_route(lg, k)
        assert np.array_equal(idx.astype(np.int32), oi), (lg, idx, oi)
        assert np.array_equal(np.isnan(w), np.isnan(ow))
        assert np.abs(np.nan_to_num(w) - np.nan_to_num(ow)).max() <= 2e-5


def test_host_route_brute_force_ties():
    rng = np.random.default_rng(7)
    for _ in range(40):
        n = int(rng.integers(8, 257))
        lg = rng.integers(-4, 4, n).astype(np.float32)
        idx, w = Q.moe_route_host(lg, 8)
        oi, ow = O.moe_route(lg, 8)
        assert np.array_equal(idx.astype(np.int32), oi)
        assert np.abs(w - ow).max() <= 2e-5


def test_host_silu_gather_rmsnorm():
    i = np.arange(513)
    g = (((i % 31).astype(np.float32) - 15) * 0.125).astype(np.float32)
    u = np.cos(i.astype(np.float32) * np.float32(0.031)).astype(np.float32)
    assert np.abs(Q.silu_mul_host(g, u) - O.silu_mul(g, u)).max() <= 2e-5
    dim, k = 257, 8
    wts = (0.1 + 0.03 * np.arange(k)).astype(np.float32)
    wts /= wts.sum()
    eo = np.sin(np.arange(k * dim, dtype=np.float32).reshape(k, dim) * np.float32(0.021))
    sh = np.cos(np.arange(dim, dtype=np.float32) * np.float32(0.019)).astype(np.float32)
    assert np.abs(Q.moe_gather_host(eo, wts, sh, 0.25) - O.moe_gather(eo, wts, sh, 0.25)).max() <= 2e-5
    assert np.abs(Q.moe_gather_host(eo, wts, None, 0.0) - O.moe_gather(eo, wts, None, 0.0)).max() <= 2e-5
    x = S.f32_normal(7, S.stream_id(0, S.K_X, 99), 2048, 1.0)
    y = Q.rmsnorm_host(x, cases.norm_w(7, 0))
    assert cases.rel_l2(y, G["rms_out"]) <= TOL


# ---- device API -------------------------------------------------------------------

def test_device_synth_matches_host_generator(torch_dev, ctx):
    torch = torch_dev
    for q in FORMATS:
        nb = 300
        buf = torch.empty(nb * S.BLOCK_BYTES[q], dtype=torch.uint8, device="cuda")
        Q.synth_blocks(buf, q, nb, 17, 1234, first=5)
        torch.cuda.synchronize()
        assert np.array_equal(buf.cpu().numpy(), S.quant_blocks(17, 1234, q, nb, start=5).reshape(-1)), q
    f = torch.empty(5000, dtype=torch.float32, device="cuda")
    Q.synth_normal(f, 5000, 0.02, 17, 99)
    torch.cuda.synchronize()
    assert np.array_equal(f.cpu().numpy(), S.f32_normal(17, 99, 5000, 0.02))
    # with a mean (norm weights N(1, 0.1)): mean + sd * z, two roundings
    Q.synth_normal(f, 5000, 0.1, 17, 98, mean=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(f.cpu().numpy(), S.f32_normal(17, 98, 5000, 0.1, mean=1.0))


@pytest.mark.parametrize("q", FORMATS)
def test_device_matvec_multi_token(torch_dev, ctx, q):
    torch = torch_dev
    rows, cols, T = 64, 2048, 4
    w = S.quant_matrix(9, 77, q, rows, cols)
    xs = np.stack([S.f32_normal(9, 78 + t, cols, 1.0) for t in range(T)])
    dw = torch.from_numpy(w).cuda()
    dx = torch.from_numpy(xs).cuda()
    for n in (1, 2, 3, 4):
        dy = torch.zeros(n, rows, dtype=torch.float32, device="cuda")
        ctx.matvec((dw.data_ptr(), q, rows, cols), dx, dy, n_tok=n)
        torch.cuda.synchronize()
        y = dy.cpu().numpy()
        for t in range(n):
            assert cases.rel_l2(y[t], O.matvec(q, w, rows, cols, xs[t])) <= TOL


@pytest.fixture(scope="module")
def layers(torch_dev, ctx):
    from qw6_amd.workload import SynthLayer
    out = {}
    for mix, seed, shared in (("q4k", 11, True), ("q4k", 13, False), ("iq2m", 21, True)):
        say("building device layer", mix, seed)
        out[(mix, seed)] = SynthLayer(ctx, seed, 0, mix, shared=shared)
    yield out
    for L in out.values():
        L.free()


def run_layer(torch, ctx, L, xs, logits=None, residual=None):
    T = xs.shape[0]
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
    didx = torch.zeros(T, L.top_k, dtype=torch.int32, device="cuda")
    dw = torch.zeros(T, L.top_k, dtype=torch.float32, device="cuda")
    dl = None if logits is None else torch.from_numpy(np.ascontiguousarray(logits)).cuda()
    dr = None if residual is None else torch.from_numpy(np.ascontiguousarray(residual)).cuda()
    ctx.moe_forward(L.desc, dx, dout, n_tok=T, logits=dl, residual=dr, idx=didx, w=dw)
    torch.cuda.synchronize()
    return dout.cpu().numpy(), didx.cpu().numpy(), dw.cpu().numpy()


def oracle_for(L, x, logits=None, router=None):
    lg = logits if logits is not None else O.matvec(0, router, L.n_experts, L.hidden, x)
    idx, _ = O.moe_route(lg, L.top_k)
    ex = [L.expert_host(e) if e in set(int(i) for i in idx) else None
          for e in range(L.n_experts)]
    ol = O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, router, ex, L.shared_host())
    return O.moe_layer(ol, x, logits=logits), cases.route_gap(lg)


@pytest.mark.parametrize("key", [("q4k", 11), ("q4k", 13), ("iq2m", 21)])
def test_layer_vs_golden(torch_dev, ctx, layers, key):
    """Device-generated layer (same seed as the fixtures) through the three
    kernels vs qw6's own qw6_apply_layer_moe output."""
    mix, seed = key
    L = layers[key]
    x = cases.token_x(seed, 0)[None]
    out, idx, w = run_layer(torch_dev, ctx, L, x)
    gk = "layer_%s_s%d%s" % (mix, seed, "" if seed != 13 else "_noshared")
    assert np.array_equal(idx[0], G[gk + "_idx"])
    assert np.abs(w[0] - G[gk + "_w"]).max() <= 2e-5
    assert cases.rel_l2(out[0], G[gk + "_out"]) <= TOL


def test_selftest_passes(torch_dev):
    """qw6_hip_selftest: every known-answer case within its tolerance."""
    assert Q.lib().qw6_hip_selftest() == 0


@pytest.mark.parametrize("mix,seed", [("q4k", 14), ("iq2m", 23)])
def test_shared_gate_layer_vs_golden(torch_dev, ctx, mix, seed):
    """The shared expert weighted by sigmoid(shared_router . x) (qw6.c:
    2267-2272): device layer, device-generated gate vector, against qw6's own
    qw6_apply_layer_moe with the same shared router."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    say("shared gate layer", mix, seed)
    L = SynthLayer(ctx, seed, 0, mix)
    try:
        sr = torch.empty(L.hidden, dtype=torch.float32, device="cuda")
        Q.synth_normal(sr, L.hidden, 0.02, seed, S.stream_id(0, S.K_SROUTER))
        host = cases.HostLayer(seed, 0, mix, shared_router=True)
        torch.cuda.synchronize()
        assert np.array_equal(sr.cpu().numpy(), host.shared_router)
        d = Q.MoeLayer.from_buffer_copy(L.desc)
        d.shared_router = sr.data_ptr()
        x = torch.from_numpy(cases.token_x(seed, 0)[None].copy()).cuda()
        out = torch.zeros_like(x)
        idx = torch.zeros(1, L.top_k, dtype=torch.int32, device="cuda")
        ctx.moe_forward(d, x, out, n_tok=1, idx=idx)
        torch.cuda.synchronize()
        gk = "layer_%s_s%d_sr" % (mix, seed)
        assert np.array_equal(idx.cpu().numpy()[0], G[gk + "_idx"])
        assert cases.rel_l2(out.cpu().numpy()[0], G[gk + "_out"]) <= TOL
    finally:
        L.free()


@pytest.mark.parametrize("key", [("q4k", 11), ("iq2m", 21)])
def test_layer_many_tokens_vs_oracle(torch_dev, ctx, layers, key):
    """Random tokens (T = 1, 2 as in MTP verification, 3) against the oracle;
    near-tie routings are counted, not failed."""
    L = layers[key]
    router = L.router_host()
    ties = 0
    for T in (1, 2, 3):
        xs = np.stack([cases.token_x(500 + T, 1, t) for t in range(T)])
        out, idx, _ = run_layer(torch_dev, ctx, L, xs)
        for t in range(T):
            (oo, oi, _), gap = oracle_for(L, xs[t], router=router)
            if gap < TIE:
                ties += 1
                continue
            assert np.array_equal(idx[t], oi)
            assert cases.rel_l2(out[t], oo) <= TOL
    assert ties <= 1


def test_layer_given_logits_and_residual(torch_dev, ctx):
    """Batched tokens with given (Zipf) router logits vs the golden fixture,
    plus the residual add (hidden = resid + ffn)."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 51, 0, "q4k", router=False)
    try:
        lg = S.zipf_logits(51, 4)
        xs = np.stack([cases.token_x(51, 0, t) for t in range(4)])
        res = np.stack([cases.token_x(52, 0, t) for t in range(4)])
        out, idx, _ = run_layer(torch_dev, ctx, L, xs, logits=lg, residual=res)
        for t in range(4):
            assert np.array_equal(idx[t], G["prefill_t%d_idx" % t])
            assert cases.rel_l2(out[t] - res[t], G["prefill_t%d_out" % t]) <= TOL
    finally:
        L.free()


def test_stack_vs_golden(torch_dev, ctx):
    """3-layer stack, 2 steps: h <- h + MoE_l(RMSNorm(h, w_l)) on the device."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    seed = 41
    Ls = [SynthLayer(ctx, seed, l, "iq2m") for l in range(3)]
    try:
        nw = [torch.from_numpy(cases.norm_w(seed, l)).cuda() for l in range(3)]
        for step in range(2):
            h = torch.from_numpy(cases.token_x(seed, 100, step)[None].copy()).cuda()
            xn = torch.empty_like(h)
            for l, L in enumerate(Ls):
                ctx.rmsnorm(h, nw[l], xn, 2048, 1)
                hn = torch.empty_like(h)
                didx = torch.zeros(1, 8, dtype=torch.int32, device="cuda")
                ctx.moe_forward(L.desc, xn, hn, n_tok=1, residual=h, idx=didx)
                torch.cuda.synchronize()
                assert np.array_equal(didx.cpu().numpy()[0], G["stack_s%d_l%d_idx" % (step, l)])
                h = hn
            assert cases.rel_l2(h.cpu().numpy()[0], G["stack_s%d_h" % step]) <= TOL
    finally:
        for L in Ls:
            L.free()


def test_graph_replay_matches_eager(torch_dev, ctx, layers):
    """The three kernels captured in a graph and replayed several times, with
    eager work in between; every replay equals the eager result."""
    torch = torch_dev
    L = layers[("q4k", 11)]
    x = torch.from_numpy(cases.token_x(11, 0)[None].copy()).cuda()
    eager = torch.zeros(1, 2048, dtype=torch.float32, device="cuda")
    ctx.moe_forward(L.desc, x, eager, n_tok=1)
    torch.cuda.synchronize()
    out = torch.zeros_like(eager)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        ctx.moe_forward(L.desc, x, out, n_tok=1, stream=s.cuda_stream)   # warm
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            ctx.moe_forward(L.desc, x, out, n_tok=1, stream=s.cuda_stream)
    for _ in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ctx.moe_forward(L.desc, x, eager, n_tok=1)
        torch.cuda.synchronize()


def test_error_paths(torch_dev, ctx, layers):
    torch = torch_dev
    L = layers[("q4k", 11)]
    x = torch.zeros(8, 2048, dtype=torch.float32, device="cuda")
    out = torch.zeros_like(x)
    with pytest.raises(Q.Qw6HipError, match="max_tokens"):
        ctx.moe_forward(L.desc, x, out, n_tok=8)
    bad = list(L.mats[0])
    bad[3] = (bad[3][0], 3, bad[3][2], bad[3][3])    # Q8_0: no decoder
    with pytest.raises(Q.Qw6HipError, match="quant"):
        ctx.experts(bad, L.mats[1], L.mats[2])
    mis = list(L.mats[0])
    mis[0] = (mis[0][0] + 2, mis[0][1], mis[0][2], mis[0][3])
    with pytest.raises(Q.Qw6HipError, match="aligned"):
        ctx.experts(mis, L.mats[1], L.mats[2])
    shp = list(L.mats[2])
    shp[1] = (shp[1][0], shp[1][1], 1024, shp[1][3])
    with pytest.raises(Q.Qw6HipError, match="shape"):
        ctx.experts(L.mats[0], L.mats[1], shp)
    # activations are read in 16-byte pieces: a pointer 4 bytes off is refused
    # on the host, before any launch (the layer's residual, the device matvec's
    # input, the output head's input and norm weight)
    buf = torch.zeros(2048 + 4, dtype=torch.float32, device="cuda")
    off = buf[1:1 + 2048]
    with pytest.raises(Q.Qw6HipError, match="aligned"):
        ctx.moe_forward(L.desc, x[:1], out[:1], n_tok=1, residual=off)
    with pytest.raises(Q.Qw6HipError, match="aligned"):
        ctx.matvec(L.mats[0][0], off, torch.zeros(512, dtype=torch.float32, device="cuda"))
    with pytest.raises(Q.Qw6HipError, match="aligned"):   # expert 0's down: 2048 x 512
        ctx.output_greedy(L.mats[2][0], off[:512], torch.zeros(2048, dtype=torch.float32, device="cuda"),
                          torch.zeros(1, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()


def test_given_logits_on_a_layer_with_router(torch_dev, ctx, layers):
    """Router logits passed in for a layer that also has a router (the logits
    win, the router is not read) on the per-token kernels, T = 1 and 3."""
    L = layers[("q4k", 11)]
    for T in (1, 3):
        lg = S.zipf_logits(81 + T, T)
        xs = np.stack([cases.token_x(81, 7, t) for t in range(T)])
        out, idx, _ = run_layer(torch_dev, ctx, L, xs, logits=lg)
        for t in range(T):
            (oo, oi, _), _ = oracle_for(L, xs[t], logits=lg[t])
            assert np.array_equal(idx[t], oi)
            assert cases.rel_l2(out[t], oo) <= TOL


def test_in_place_residual_update(torch_dev, ctx, layers):
    """hidden <- hidden + MoE(rmsnorm(hidden)) with x, residual and out the same
    buffer (qw6.c:2475-2484 updates the hidden state in place) equals the call
    with separate buffers, for T = 1 and 3."""
    torch = torch_dev
    L = layers[("q4k", 11)]
    nw = torch.from_numpy(cases.norm_w(11, 0)).cuda()
    layer = Q.MoeLayer.from_buffer_copy(L.desc)
    layer.norm_w, layer.norm_eps = nw.data_ptr(), 1e-6
    for T in (1, 3):
        xs = np.stack([cases.token_x(91, 3, t) for t in range(T)])
        h = torch.from_numpy(xs).cuda()
        ref = torch.empty_like(h)
        ctx.moe_forward(layer, h, ref, n_tok=T, residual=h)
        torch.cuda.synchronize()
        ctx.moe_forward(layer, h, h, n_tok=T, residual=h)
        torch.cuda.synchronize()
        assert torch.equal(h, ref)


@pytest.mark.parametrize("mix", ["q4k", "iq2m"])
def test_layer_other_shape_vs_oracle(torch_dev, ctx, mix):
    """hidden 1024, inter 256, 64 experts, top-4 (the unit-count-generic
    kernels, fewer experts, top_k < 8): T = 1 and 3 with the router GEMV on the
    device, against the oracle."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 31, 0, mix, hidden=1024, inter=256, n_experts=64, top_k=4)
    try:
        router = L.router_host()
        checked = 0
        for T in (1, 3):
            xs = np.stack([cases.token_x(31, 2, t, hidden=1024) for t in range(T)])
            out, idx, _ = run_layer(torch_dev, ctx, L, xs)
            for t in range(T):
                (oo, oi, _), gap = oracle_for(L, xs[t], router=router)
                if gap < TIE:
                    continue
                assert np.array_equal(idx[t], oi)
                assert cases.rel_l2(out[t], oo) <= TOL
                checked += 1
        assert checked >= 3
    finally:
        L.free()


def test_zero_tokens_is_a_no_op(torch_dev, ctx, layers):
    torch = torch_dev
    L = layers[("q4k", 11)]
    x = torch.zeros(1, 2048, dtype=torch.float32, device="cuda")
    out = torch.full((1, 2048), 7.0, dtype=torch.float32, device="cuda")
    ctx.moe_forward(L.desc, x, out, n_tok=0)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
