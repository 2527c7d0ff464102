"""Small-batch MFMA kernels (k_mx_gate_up / k_mx_down; qw6_hip_set_mode 3)
against the oracle, through the C ABI, and the automatic choice at the same
token counts (the fp32 kernels, one grid row per token).

Same bars as the fp32 per-token kernels: expert indices bit-exact, outputs
rel-L2 <= 1e-5 (the activations enter as three bf16 parts and the weights as
exact integer codes, so the products carry fp32 precision). Tokens whose
8th/9th router logits are closer than 1e-4 are skipped (the GPU and the CPU
sum the router dot product in different orders).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import cases
import oracle as O
import qw6_amd as Q
from qw6_amd import synth as S

pytestmark = pytest.mark.gpu

TOL = 1e-5
TIE = 1e-4
MIXES = ["q4k", "iq2m", "q5k", "q6q4", "iq2a", "iq2b"]


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
    c = Q.Context(0, max_tokens=16)
    yield c
    c.close()


def run(torch, ctx, L, xs, mode, logits=None, residual=None, layer=None):
    T = xs.shape[0]
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
    didx = torch.zeros(T, L.top_k, dtype=torch.int32, device="cuda")
    dl = None if logits is None else torch.from_numpy(np.ascontiguousarray(logits)).cuda()
    dr = None if residual is None else torch.from_numpy(np.ascontiguousarray(residual)).cuda()
    ctx.set_mode(mode)
    try:
        ctx.moe_forward(L.desc if layer is None else layer, dx, dout, n_tok=T, logits=dl,
                        residual=dr, idx=didx)
        torch.cuda.synchronize()
    finally:
        ctx.set_mode(0)
    return dout.cpu().numpy(), didx.cpu().numpy()


def oracle_token(L, x, router=None, logits=None):
    lg = logits if logits is not None else O.matvec(0, router, L.n_experts, L.hidden, x)
    idx, _ = O.moe_route(lg, L.top_k)
    sel = set(int(i) for i in idx)
    ex = [L.expert_host(e) if e in sel else None for e in range(L.n_experts)]
    ol = O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, router, ex, L.shared_host())
    out, oi, _ = O.moe_layer(ol, x, logits=logits)
    return out, oi, cases.route_gap(lg, L.top_k)


def check_tokens(L, xs, out, idx, router=None, logits=None, resid=None, tol=None):
    """Every token against the oracle (rel-L2 <= tol, default TOL); returns
    how many were compared."""
    n = 0
    for t in range(xs.shape[0]):
        oo, oi, gap = oracle_token(L, xs[t], router=router,
                                   logits=None if logits is None else logits[t])
        if gap < TIE:
            say("near tie skipped, token", t)
            continue
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        got = out[t] if resid is None else out[t] - resid[t]
        err = cases.rel_l2(got, oo)
        assert err <= (TOL if tol is None else tol), (t, err)
        n += 1
    return n


@pytest.mark.parametrize("mix", MIXES)
def test_mx_layer_vs_oracle(torch_dev, ctx, mix):
    """Every format mix (routed and shared formats differ in several), T = 1..4
    through the MFMA kernels with the router GEMV on the device."""
    from qw6_amd.workload import SynthLayer
    say("mx layer", mix)
    L = SynthLayer(ctx, 61, 0, mix)
    try:
        router = L.router_host()
        n = 0
        for T in (1, 2, 3, 4):
            xs = np.stack([cases.token_x(610 + T, 1, t) for t in range(T)])
            out, idx = run(torch_dev, ctx, L, xs, 3)
            n += check_tokens(L, xs, out, idx, router=router)
        assert n >= 8
    finally:
        L.free()


def test_mx_agrees_with_fp32_kernels(torch_dev, ctx):
    """The MFMA and fp32 per-token kernels on the same tokens: identical
    routing, outputs within twice the oracle bar of each other."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 62, 0, "iq2m")
    try:
        for T in (1, 2, 4):
            xs = np.stack([cases.token_x(620 + T, 1, t) for t in range(T)])
            o1, i1 = run(torch_dev, ctx, L, xs, 1)
            o3, i3 = run(torch_dev, ctx, L, xs, 3)
            assert np.array_equal(i1, i3)
            for t in range(T):
                assert cases.rel_l2(o3[t], o1[t]) <= 2 * TOL
    finally:
        L.free()


@pytest.mark.parametrize("mix", ["q4k", "iq2b"])
def test_mx_other_shape_vs_oracle(torch_dev, ctx, mix):
    """hidden 1024, inter 256, 64 experts, top-4: four 256-column blocks per
    gate/up row (four waves), one per down row; T = 1..4."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 63, 0, mix, hidden=1024, inter=256, n_experts=64, top_k=4)
    try:
        router = L.router_host()
        n = 0
        for T in (1, 2, 3, 4):
            xs = np.stack([cases.token_x(630 + T, 2, t, hidden=1024) for t in range(T)])
            out, idx = run(torch_dev, ctx, L, xs, 3)
            n += check_tokens(L, xs, out, idx, router=router)
        assert n >= 8
    finally:
        L.free()


@pytest.mark.parametrize("hidden,mix", [(512, "q4k"), (256, "iq2b"), (512, "iq2a")])
def test_mx_narrow_hidden_vs_oracle(torch_dev, ctx, hidden, mix):
    """hidden 256 / 512: one or two 256-column blocks per gate/up row, fewer
    than the 4 tokens of a launch; the gate/up kernel still runs one routing
    wave per token. T = 1..4, inter 256, 32 experts."""
    from qw6_amd.workload import SynthLayer
    say("mx narrow", hidden, mix)
    L = SynthLayer(ctx, 69, 0, mix, hidden=hidden, inter=256, n_experts=32)
    try:
        router = L.router_host()
        n = 0
        for T in (1, 2, 3, 4):
            xs = np.stack([cases.token_x(690 + T, 2, t, hidden=hidden) for t in range(T)])
            out, idx = run(torch_dev, ctx, L, xs, 3)
            n += check_tokens(L, xs, out, idx, router=router)
        assert n >= 8
    finally:
        L.free()


@pytest.mark.parametrize("hidden,inter,n_exp,top_k,mix",
                         [(512, 256, 32, 8, "q4k"), (1024, 256, 64, 4, "iq2m"),
                          (256, 256, 32, 8, "iq2b"), (2048, 1024, 64, 6, "q5k")])
def test_token_rows_other_shapes_vs_oracle(torch_dev, ctx, hidden, inter, n_exp, top_k, mix):
    """The fp32 kernels' launches of several tokens (one grid row per token,
    mode 1) on other layer shapes: 256-2048 columns per gate/up row (the
    generic row-length instantiations), top_k 4 and 6 (per-token slot tables
    and mid blocks of top_k + 1 rows, down workgroups of fewer waves), a
    Q5_K layer. T = 2, 5 and 16 against the oracle."""
    from qw6_amd.workload import SynthLayer
    say("token rows", hidden, inter, n_exp, top_k, mix)
    L = SynthLayer(ctx, 73, 0, mix, hidden=hidden, inter=inter, n_experts=n_exp, top_k=top_k)
    try:
        router = L.router_host()
        n = 0
        for T in (2, 5, 16):
            xs = np.stack([cases.token_x(730 + T, 2, t, hidden=hidden) for t in range(T)])
            out, idx = run(torch_dev, ctx, L, xs, 1)
            n += check_tokens(L, xs, out, idx, router=router)
        assert n >= 18
    finally:
        L.free()


@pytest.mark.parametrize("mix", ["q4k", "iq2m"])
def test_auto_switch_points_vs_oracle(torch_dev, mix):
    """The automatic mode on both sides of its switch to the grouped kernels
    (17 tokens for a Q4_K / Q6_K layer, 16 for one holding IQ formats): 15,
    16 and 17 tokens against the oracle, at the fp32 bar (the grouped kernels
    take three activation parts below 64 tokens)."""
    from qw6_amd.workload import SynthLayer
    c = Q.Context(0, max_tokens=17)
    L = SynthLayer(c, 75, 0, mix)
    try:
        router = L.router_host()
        n = 0
        for T in (15, 16, 17):
            say("auto switch", mix, T)
            xs = np.stack([cases.token_x(750 + T, 2, t) for t in range(T)])
            out, idx = run(torch_dev, c, L, xs, 0)
            n += check_tokens(L, xs, out, idx, router=router)
        assert n >= 40
    finally:
        L.free()
        c.close()


def test_mx_no_shared_given_logits_residual(torch_dev, ctx):
    """No shared expert, router logits given (Zipf), residual added: the router
    kernel then only writes the operands (mode 3), or does not run (the fp32
    kernels, one grid row per token, at 3 and 9 tokens)."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 64, 0, "q4k", shared=False, router=False)
    try:
        for T, mode in ((1, 3), (3, 3), (3, 1), (9, 1)):
            lg = S.zipf_logits(640 + T, T)
            xs = np.stack([cases.token_x(640 + T, 1, t) for t in range(T)])
            res = np.stack([cases.token_x(641 + T, 1, t) for t in range(T)])
            out, idx = run(torch_dev, ctx, L, xs, mode, logits=lg, residual=res)
            assert check_tokens(L, xs, out, idx, logits=lg, resid=res) == T
    finally:
        L.free()


def test_mx_norm_in_place_matches_separate_buffers(torch_dev, ctx):
    """RMSNorm inside the call and x = residual = out (in place), T = 2 and 4:
    equal to the call with separate buffers, and to the oracle on the
    normalised input."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 65, 0, "iq2m")
    try:
        nw_h = cases.norm_w(65, 0)
        nw = torch.from_numpy(nw_h).cuda()
        layer = Q.MoeLayer.from_buffer_copy(L.desc)
        layer.norm_w, layer.norm_eps = nw.data_ptr(), 1e-6
        router = L.router_host()
        ctx.set_mode(3)
        try:
            for T in (2, 4):
                xs = np.stack([cases.token_x(650 + T, 3, t) for t in range(T)])
                h = torch.from_numpy(xs).cuda()
                ref = torch.empty_like(h)
                ctx.moe_forward(layer, h, ref, n_tok=T, residual=h)
                torch.cuda.synchronize()
                ctx.moe_forward(layer, h, h, n_tok=T, residual=h)
                torch.cuda.synchronize()
                assert torch.equal(h, ref)
                xn = np.stack([O.rmsnorm(xs[t], nw_h, 1e-6) for t in range(T)])
                out = ref.cpu().numpy()
                n = 0
                for t in range(T):
                    oo, _, gap = oracle_token(L, xn[t], router=router)
                    if gap < TIE:
                        continue
                    assert cases.rel_l2(out[t] - xs[t], oo) <= TOL
                    n += 1
                assert n >= T - 1
        finally:
            ctx.set_mode(0)
    finally:
        L.free()


def test_mx_graph_replay_matches_eager(torch_dev, ctx):
    """T = 2 through the MFMA kernels captured once and replayed several times
    with eager calls between: every replay equals the eager result bit for
    bit (fixed summation orders, no atomics)."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 66, 0, "q4k")
    try:
        xs = np.stack([cases.token_x(66, 1, t) for t in range(2)])
        x = torch.from_numpy(xs).cuda()
        ctx.set_mode(3)
        try:
            eager = torch.zeros(2, 2048, dtype=torch.float32, device="cuda")
            ctx.moe_forward(L.desc, x, eager, n_tok=2)
            torch.cuda.synchronize()
            out = torch.zeros_like(eager)
            s = torch.cuda.Stream()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                ctx.moe_forward(L.desc, x, out, n_tok=2, stream=s.cuda_stream)
                torch.cuda.synchronize()
                with torch.cuda.graph(g, stream=s):
                    ctx.moe_forward(L.desc, x, out, n_tok=2, stream=s.cuda_stream)
            for _ in range(4):
                out.zero_()
                g.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, eager)
                ctx.moe_forward(L.desc, x, eager, n_tok=2)
                torch.cuda.synchronize()
        finally:
            ctx.set_mode(0)
    finally:
        L.free()


def test_auto_mode_mixed_chunks_vs_oracle(torch_dev, ctx):
    """Calls of 5-7 tokens on a mixed-format layer (IQ2_XXS gate/up, IQ3_S /
    IQ2_S down), through the call without allocation (which never takes the
    grouped kernels) and the automatic path: both run one launch of the fp32
    kernels, one grid row per token (the grouped kernels start at 16 tokens
    for layers holding IQ formats). A uniform Q4_K layer under the per-token
    mode (1) takes 5 tokens in one launch too."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 67, 0, "iq2m")
    try:
        router = L.router_host()
        n = 0
        for T in (5, 6, 7):
            xs = np.stack([cases.token_x(670 + T, 1, t) for t in range(T)])
            dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
            dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
            didx = torch.zeros(T, L.top_k, dtype=torch.int32, device="cuda")
            ctx.moe_forward_noalloc(L.desc, dx, dout, n_tok=T, idx=didx)
            torch.cuda.synchronize()
            n += check_tokens(L, xs, dout.cpu().numpy(), didx.cpu().numpy(), router=router)
            out, idx = run(torch_dev, ctx, L, xs, 0)
            n += check_tokens(L, xs, out, idx, router=router, tol=1e-5)
        assert n >= 30
    finally:
        L.free()
    L = SynthLayer(ctx, 69, 0, "q4k")
    try:
        router = L.router_host()
        xs = np.stack([cases.token_x(695, 1, t) for t in range(5)])
        out, idx = run(torch_dev, ctx, L, xs, 1)
        assert check_tokens(L, xs, out, idx, router=router) >= 4
    finally:
        L.free()


def test_auto_mode_mixed_formats_vs_oracle(torch_dev, ctx):
    """Automatic path selection on a mixed-format layer (IQ2_XXS routed with a
    Q4_K shared gate/up, IQ3_S / IQ2_S routed down with a Q6_K shared down):
    2-4 tokens take the fp32 kernels' per-matrix format dispatch, one grid row
    per token."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 68, 0, "iq2m")
    try:
        router = L.router_host()
        n = 0
        for T in (2, 3, 4):
            xs = np.stack([cases.token_x(680 + T, 1, t) for t in range(T)])
            out, idx = run(torch_dev, ctx, L, xs, 0)
            n += check_tokens(L, xs, out, idx, router=router)
        assert n >= 8
    finally:
        L.free()
