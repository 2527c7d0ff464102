"""The batched (grouped bf16-MFMA) MoE path against the oracle, through the
C ABI. Bars: expert indices exact for given router logits. Outputs: calls of
64 tokens or more, rel-L2 <= 2e-3 per token (the bf16-MFMA bar) with a mean
<= 1e-4; calls of fewer tokens (where the automatic path also takes these
kernels) are held to the fp32 bar, rel-L2 <= 1e-5 per token: they split the
activations into three bf16 parts (hi, mid, lo: 24 significant bits) beside
the exact integer weight codes and fp32 scales, where calls of 64 tokens or
more use two (hi, lo). The full T = 512 batch is
checked against the per-token fp32 kernels of the same library (a
size-independent consistency check) and on a sample of tokens against the
oracle.
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

TOL_BF16 = 2e-3
TOL_MEAN = 1e-4
TOL_SMALL = 1e-5        # fewer than 64 tokens: per token (three activation parts)
TOL_SMALL_MEAN = 1e-5   # and in the mean


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
    c = Q.Context(0, max_tokens=512)
    yield c
    c.close()


@pytest.fixture(scope="module")
def layer(torch_dev, ctx):
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 61, 0, "q4k")
    yield L
    L.free()


def run(torch, ctx, L, xs, logits=None, residual=None, mode=2):
    T = xs.shape[0]
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
    didx = torch.zeros(T, L.top_k, dtype=torch.int32, device="cuda")
    dw = torch.zeros(T, L.top_k, dtype=torch.float32, device="cuda")
    dl = None if logits is None else torch.from_numpy(np.ascontiguousarray(logits)).cuda()
    dr = None if residual is None else torch.from_numpy(np.ascontiguousarray(residual)).cuda()
    ctx.set_mode(mode)
    try:
        ctx.moe_forward(L.desc, dx, dout, n_tok=T, logits=dl, residual=dr, idx=didx, w=dw)
        torch.cuda.synchronize()
    finally:
        ctx.set_mode(0)
    return dout.cpu().numpy(), didx.cpu().numpy(), dw.cpu().numpy()


def oracle_tokens(L, xs, lg, tokens, router=None):
    need = set()
    for t in tokens:
        idx, _ = O.moe_route(lg[t], L.top_k)
        need.update(int(i) for i in idx)
    ex = [L.expert_host(e) if e in need else None for e in range(L.n_experts)]
    ol = O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, router, ex, L.shared_host())
    return {t: O.moe_layer(ol, xs[t], logits=None if router is not None else lg[t], nthreads=8)
            for t in tokens}


def test_grouped_given_logits_vs_oracle(torch_dev, ctx, layer):
    """T = 64 tokens, Zipf(1.1)-skewed given logits, shared expert, residual."""
    T = 64
    lg = S.zipf_logits(61, T)
    xs = np.stack([cases.token_x(61, 3, t) for t in range(T)])
    res = np.stack([cases.token_x(62, 3, t) for t in range(T)])
    say("grouped T=%d" % T)
    out, idx, w = run(torch_dev, ctx, layer, xs, logits=lg, residual=res)
    want = oracle_tokens(layer, xs, lg, range(T))
    rels = []
    for t in range(T):
        oo, oi, ow = want[t]
        assert np.array_equal(idx[t], oi), t
        assert np.abs(w[t] - ow).max() <= 2e-5
        rels.append(cases.rel_l2(out[t] - res[t], oo))
    say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
    assert max(rels) <= TOL_BF16
    assert np.mean(rels) <= TOL_MEAN


@pytest.mark.parametrize("mix", ["q5k", "q6q4", "iq2a", "iq2b"])
def test_grouped_other_formats_vs_oracle(torch_dev, ctx, mix):
    """The other formats through the grouped kernels (T = 48, given logits):
    Q5_K throughout; Q6_K gate/up with Q4_K down; IQ2_XXS gate/up with IQ3_S
    down and a Q4_K / Q6_K shared expert (its own launches); IQ2_S throughout
    with an IQ3_S / IQ2_XXS shared expert."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 71, 0, mix)
    try:
        T = 48
        lg = S.zipf_logits(72, T)
        xs = np.stack([cases.token_x(71, 5, t) for t in range(T)])
        say("grouped %s T=%d" % (mix, T))
        out, idx, _ = run(torch_dev, ctx, L, xs, logits=lg)
        toks = list(range(0, T, 3))
        want = oracle_tokens(L, xs, lg, toks)
        rels = []
        for t in toks:
            oo, oi, _ = want[t]
            assert np.array_equal(idx[t], oi), t
            rels.append(cases.rel_l2(out[t], oo))
        say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_SMALL
        assert np.mean(rels) <= TOL_SMALL_MEAN
    finally:
        L.free()


def test_grouped_other_shape_vs_oracle(torch_dev, ctx):
    """hidden 1024, inter 256, 64 experts, top-4 through the grouped kernels
    (T = 40, given logits, shared expert), against the oracle."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 33, 0, "q4k", hidden=1024, inter=256, n_experts=64, top_k=4)
    try:
        T = 40
        lg = S.zipf_logits(34, T, n_experts=64)
        xs = np.stack([cases.token_x(33, 4, t, hidden=1024) for t in range(T)])
        say("grouped 1024x256 E64 k4 T=%d" % T)
        out, idx, _ = run(torch_dev, ctx, L, xs, logits=lg)
        toks = list(range(0, T, 4))
        want = oracle_tokens(L, xs, lg, toks)
        rels = []
        for t in toks:
            oo, oi, _ = want[t]
            assert np.array_equal(idx[t], oi), t
            rels.append(cases.rel_l2(out[t], oo))
        say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_SMALL
        assert np.mean(rels) <= TOL_SMALL_MEAN
    finally:
        L.free()


@pytest.mark.parametrize("T", [40, 96])
def test_grouped_shared_gate_vs_oracle(torch_dev, ctx, T):
    """The shared expert weighted by sigmoid(shared_router . x) (qw6.c:
    2267-2285) on the batched path: the gate is a dot product split over the
    route kernel's four waves, then the weight rides with the shared entries
    through the down kernel. Router GEMV on; every token against the oracle."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    say("grouped shared gate", T)
    L = SynthLayer(ctx, 73, 0, "q4k")
    try:
        sr = S.f32_normal(73, S.stream_id(0, S.K_SROUTER), L.hidden, 0.05)
        dsr = torch.from_numpy(sr).cuda()
        desc = Q.make_layer(L.hidden, L.inter, L.top_k, L.experts, router=L.router,
                            shared=L.shared, shared_router=dsr)
        xs = np.stack([cases.token_x(73, 6, t) for t in range(T)])
        dx = torch.from_numpy(xs).cuda()
        dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
        didx = torch.zeros(T, L.top_k, dtype=torch.int32, device="cuda")
        ctx.set_mode(2)
        try:
            ctx.moe_forward(desc, dx, dout, n_tok=T, idx=didx)
            torch.cuda.synchronize()
        finally:
            ctx.set_mode(0)
        out, idx = dout.cpu().numpy(), didx.cpu().numpy()
        router = L.router_host()
        lg = np.stack([O.matvec(0, router, L.n_experts, L.hidden, xs[t]) for t in range(T)])
        need = set()
        for t in range(T):
            need.update(int(i) for i in O.moe_route(lg[t], L.top_k)[0])
        ex = [L.expert_host(e) if e in need else None for e in range(L.n_experts)]
        ol = O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, router, ex, L.shared_host(), sr)
        gates = 1.0 / (1.0 + np.exp(-(xs.astype(np.float64) @ sr.astype(np.float64))))
        assert gates.min() < 0.45 and gates.max() > 0.55   # the gate weights differ by token
        ties, rels = 0, []
        for t in range(T):
            oo, oi, _ = O.moe_layer(ol, xs[t], nthreads=8)
            if cases.route_gap(lg[t]) < 1e-4:
                ties += 1
                continue
            assert np.array_equal(idx[t], oi), t
            rels.append(cases.rel_l2(out[t], oo))
        assert ties <= 1
        tol, tol_mean = (TOL_SMALL, TOL_SMALL_MEAN) if T < 64 else (TOL_BF16, TOL_MEAN)
        say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= tol and np.mean(rels) <= tol_mean, (max(rels), np.mean(rels))
    finally:
        L.free()


def test_grouped_router_and_norm_vs_oracle(torch_dev, ctx):
    """Router GEMV and the fused RMSNorm on the batched path (T = 40)."""
    torch = torch_dev
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 71, 0, "q4k")
    try:
        T = 40
        nw = cases.norm_w(71, 0)
        dnw = torch.from_numpy(nw).cuda()
        desc = Q.make_layer(L.hidden, L.inter, L.top_k, L.experts, router=L.router,
                            shared=L.shared, norm_w=dnw, norm_eps=1e-6)
        xs = np.stack([cases.token_x(71, 4, t) for t in range(T)])
        dx = torch.from_numpy(xs).cuda()
        dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
        didx = torch.zeros(T, L.top_k, dtype=torch.int32, device="cuda")
        ctx.set_mode(2)
        try:
            ctx.moe_forward(desc, dx, dout, n_tok=T, idx=didx)
            torch.cuda.synchronize()
        finally:
            ctx.set_mode(0)
        out, idx = dout.cpu().numpy(), didx.cpu().numpy()
        router = L.router_host()
        xn = np.stack([O.rmsnorm(xs[t], nw) for t in range(T)])
        lg = np.stack([O.matvec(0, router, L.n_experts, L.hidden, xn[t]) for t in range(T)])
        want = oracle_tokens(L, xn, lg, range(T), router=router)
        ties, rels = 0, []
        for t in range(T):
            oo, oi, _ = want[t]
            if cases.route_gap(lg[t]) < 1e-4:
                ties += 1
                continue
            assert np.array_equal(idx[t], oi), t
            rels.append(cases.rel_l2(out[t], oo))
        assert ties <= 1
        say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_SMALL and np.mean(rels) <= TOL_SMALL_MEAN, (max(rels), np.mean(rels))
    finally:
        L.free()


def test_grouped_full_batch_vs_per_token_kernels_and_oracle(torch_dev, ctx, layer):
    """T = 512 (the prefill workload): grouped result vs the fp32 per-token
    kernels for every token, and vs the oracle on a sample of tokens."""
    T = 512
    lg = S.zipf_logits(63, T)
    xs = np.stack([cases.token_x(63, 5, t) for t in range(T)])
    g_out, g_idx, _ = run(torch_dev, ctx, layer, xs, logits=lg, mode=2)
    d_out, d_idx, _ = run(torch_dev, ctx, layer, xs, logits=lg, mode=1)
    assert np.array_equal(g_idx, d_idx)
    rels = [cases.rel_l2(g_out[t], d_out[t]) for t in range(T)]
    say("T=512 grouped vs per-token: max %.2e mean %.2e" % (max(rels), np.mean(rels)))
    assert max(rels) <= TOL_BF16 and np.mean(rels) <= TOL_MEAN
    sample = [0, 1, 2, 77, 255, 256, 400, 511]
    want = oracle_tokens(layer, xs, lg, sample)
    for t in sample:
        oo, oi, _ = want[t]
        assert np.array_equal(g_idx[t], oi)
        assert cases.rel_l2(g_out[t], oo) <= TOL_BF16
        assert cases.rel_l2(d_out[t], oo) <= 1e-5


def test_grouped_long_batch_vs_per_token_kernels_and_oracle(torch_dev):
    """T = 1500, a long prompt: not a multiple of the 16-entry tile, and its
    12,000 (token, k) pairs take k_pre_sort three passes over its registers
    (4,096 pairs a pass). Grouped result vs the fp32 per-token kernels for
    every token (indices and gate weights equal), and vs the oracle on a
    sample of tokens, in a context sized for it."""
    from qw6_amd.workload import SynthLayer
    c = Q.Context(0, max_tokens=1500)
    L = SynthLayer(c, 62, 0, "q4k")
    try:
        T = 1500
        lg = S.zipf_logits(64, T)
        xs = np.stack([cases.token_x(64, 5, t) for t in range(T)])
        g_out, g_idx, g_w = run(torch_dev, c, L, xs, logits=lg, mode=2)
        d_out, d_idx, d_w = run(torch_dev, c, L, xs, logits=lg, mode=1)
        assert np.array_equal(g_idx, d_idx)
        assert np.abs(g_w - d_w).max() <= 2e-6
        rels = [cases.rel_l2(g_out[t], d_out[t]) for t in range(T)]
        say("T=1500 grouped vs per-token: max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_BF16 and np.mean(rels) <= TOL_MEAN
        sample = [0, 1, 511, 512, 1023, 1024, 1499]
        want = oracle_tokens(L, xs, lg, sample)
        for t in sample:
            oo, oi, _ = want[t]
            assert np.array_equal(g_idx[t], oi)
            assert cases.rel_l2(g_out[t], oo) <= TOL_BF16
            assert cases.rel_l2(d_out[t], oo) <= 1e-5
    finally:
        L.free()
        c.close()


def test_grouped_mixed_formats_vs_oracle(torch_dev, ctx):
    """Experts of different formats in one layer (qw6.h:160-162): IQ2_XXS
    gate/up, IQ3_S downs for even and IQ2_S downs for odd experts, shared
    expert Q4_K / Q6_K -- the down contraction runs as one grouped launch per
    format (IQ3_S, IQ2_S, Q6_K). T = 64 against the oracle; T = 512 against
    the fp32 per-token kernels for every token and the oracle on a sample."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 66, 0, "iq2m")
    try:
        T = 64
        lg = S.zipf_logits(66, T)
        xs = np.stack([cases.token_x(66, 1, t) for t in range(T)])
        res = np.stack([cases.token_x(66, 2, t) for t in range(T)])
        say("mixed formats grouped T=%d" % T)
        out, idx, w = run(torch_dev, ctx, L, xs, logits=lg, residual=res)
        want = oracle_tokens(L, xs, lg, range(T))
        rels = []
        for t in range(T):
            oo, oi, ow = want[t]
            assert np.array_equal(idx[t], oi), t
            assert np.abs(w[t] - ow).max() <= 2e-5
            rels.append(cases.rel_l2(out[t] - res[t], oo))
        say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_BF16 and np.mean(rels) <= TOL_MEAN
        T = 512
        lg = S.zipf_logits(67, T)
        xs = np.stack([cases.token_x(67, 3, t) for t in range(T)])
        say("mixed formats grouped T=%d" % T)
        g_out, g_idx, _ = run(torch_dev, ctx, L, xs, logits=lg, mode=2)
        d_out, d_idx, _ = run(torch_dev, ctx, L, xs, logits=lg, mode=1)
        assert np.array_equal(g_idx, d_idx)
        rels = [cases.rel_l2(g_out[t], d_out[t]) for t in range(T)]
        say("T=512 mixed grouped vs per-token: max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_BF16 and np.mean(rels) <= TOL_MEAN
        sample = [0, 5, 131, 300, 511]
        want = oracle_tokens(L, xs, lg, sample)
        for t in sample:
            oo, oi, _ = want[t]
            assert np.array_equal(g_idx[t], oi)
            assert cases.rel_l2(g_out[t], oo) <= TOL_BF16
            assert cases.rel_l2(d_out[t], oo) <= 1e-5
    finally:
        L.free()


@pytest.mark.parametrize("mix", ["iqgu", "q5q4"])
def test_mixed_gate_up_formats_vs_oracle(torch_dev, ctx, mix):
    """Routed experts whose gate/up formats differ (qw6.h:160-162): IQ2_XXS /
    IQ3_S gate/up by expert parity (downs IQ3_S / IQ2_XXS), and Q5_K / Q4_K
    gate/up (downs Q6_K), whose grouped contractions are in different
    occupancy classes and so run as separate launches. Grouped: T = 64
    against the oracle, T = 512 against the fp32 per-token kernels and an
    oracle sample. Per-token paths (automatic choice): T = 1-4 against the
    oracle at the fp32 bar."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 68, 0, mix)
    try:
        T = 64
        lg = S.zipf_logits(68, T)
        xs = np.stack([cases.token_x(68, 1, t) for t in range(T)])
        say("mixed gate/up %s grouped T=%d" % (mix, T))
        out, idx, w = run(torch_dev, ctx, L, xs, logits=lg)
        want = oracle_tokens(L, xs, lg, range(T))
        rels = []
        for t in range(T):
            oo, oi, ow = want[t]
            assert np.array_equal(idx[t], oi), t
            assert np.abs(w[t] - ow).max() <= 2e-5
            rels.append(cases.rel_l2(out[t], oo))
        say("rel-L2 max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_BF16 and np.mean(rels) <= TOL_MEAN
        for Tp in (1, 2, 3, 4):
            say("mixed gate/up %s per-token T=%d" % (mix, Tp))
            o2, i2, _ = run(torch_dev, ctx, L, xs[:Tp], logits=lg[:Tp], mode=0)
            for t in range(Tp):
                oo, oi, _ = want[t]
                assert np.array_equal(i2[t], oi), (Tp, t)
                assert cases.rel_l2(o2[t], oo) <= 1e-5, (Tp, t)
        T = 512
        lg = S.zipf_logits(69, T)
        xs = np.stack([cases.token_x(69, 3, t) for t in range(T)])
        say("mixed gate/up %s grouped T=%d" % (mix, T))
        g_out, g_idx, _ = run(torch_dev, ctx, L, xs, logits=lg, mode=2)
        d_out, d_idx, _ = run(torch_dev, ctx, L, xs, logits=lg, mode=1)
        assert np.array_equal(g_idx, d_idx)
        rels = [cases.rel_l2(g_out[t], d_out[t]) for t in range(T)]
        say("T=512 grouped vs per-token: max %.2e mean %.2e" % (max(rels), np.mean(rels)))
        assert max(rels) <= TOL_BF16 and np.mean(rels) <= TOL_MEAN
        sample = [0, 77, 255, 511]
        want = oracle_tokens(L, xs, lg, sample)
        for t in sample:
            oo, oi, _ = want[t]
            assert np.array_equal(g_idx[t], oi)
            assert cases.rel_l2(g_out[t], oo) <= TOL_BF16
            assert cases.rel_l2(d_out[t], oo) <= 1e-5
    finally:
        L.free()


def test_grouped_small_batch_vs_golden(torch_dev, ctx):
    """The 4-token golden fixture (qw6's own layer on Zipf logits, with a
    residual) through the grouped kernels."""
    import test_gpu as TG
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 51, 0, "q4k", router=False)
    try:
        lg = S.zipf_logits(51, 4)
        xs = np.stack([cases.token_x(51, 0, t) for t in range(4)])
        res = np.stack([cases.token_x(52, 0, t) for t in range(4)])
        out, idx, _ = run(torch_dev, ctx, L, xs, logits=lg, residual=res)
        for t in range(4):
            assert np.array_equal(idx[t], TG.G["prefill_t%d_idx" % t])
            assert cases.rel_l2(out[t] - res[t], TG.G["prefill_t%d_out" % t]) <= TOL_SMALL
    finally:
        L.free()


def test_grouped_graph_replay(torch_dev, ctx, layer):
    """The batched kernels captured in a graph, replayed with eager work in
    between: every replay equals the eager result."""
    torch = torch_dev
    T = 96
    lg = torch.from_numpy(S.zipf_logits(65, T)).cuda()
    x = torch.from_numpy(np.stack([cases.token_x(65, 6, t) for t in range(T)])).cuda()
    eager = torch.zeros(T, layer.hidden, dtype=torch.float32, device="cuda")
    ctx.set_mode(2)
    try:
        ctx.moe_forward(layer.desc, x, eager, n_tok=T, logits=lg)
        torch.cuda.synchronize()
        out = torch.zeros_like(eager)
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            ctx.moe_forward(layer.desc, x, out, n_tok=T, logits=lg, stream=s.cuda_stream)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                ctx.moe_forward(layer.desc, x, out, n_tok=T, logits=lg, stream=s.cuda_stream)
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            ctx.moe_forward(layer.desc, x, eager, n_tok=T, logits=lg)
            torch.cuda.synchronize()
    finally:
        ctx.set_mode(0)


def test_grouped_format_groups_graph_replay(torch_dev, ctx):
    """A layer whose shared expert has formats no routed expert has and whose
    downs mix IQ3_S and IQ2_S (several format groups per matrix kind): eager
    calls agree bitwise with each other and with every replay of the captured
    graph, and the output matches the oracle on a sample of tokens."""
    from qw6_amd.workload import SynthLayer
    torch = torch_dev
    L = SynthLayer(ctx, 68, 0, "iq2m")
    try:
        T = 96
        lg_h = S.zipf_logits(69, T)
        xs = np.stack([cases.token_x(68, 6, t) for t in range(T)])
        lg = torch.from_numpy(lg_h).cuda()
        x = torch.from_numpy(xs).cuda()
        eager = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
        again = torch.zeros_like(eager)
        ctx.set_mode(2)
        try:
            ctx.moe_forward(L.desc, x, eager, n_tok=T, logits=lg)
            ctx.moe_forward(L.desc, x, again, n_tok=T, logits=lg)
            torch.cuda.synchronize()
            assert torch.equal(again, eager)
            out = torch.zeros_like(eager)
            s = torch.cuda.Stream()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                ctx.moe_forward(L.desc, x, out, n_tok=T, logits=lg, stream=s.cuda_stream)
                torch.cuda.synchronize()
                with torch.cuda.graph(g, stream=s):
                    ctx.moe_forward(L.desc, x, out, n_tok=T, logits=lg, stream=s.cuda_stream)
            for _ in range(3):
                out.zero_()
                g.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, eager)
                ctx.moe_forward(L.desc, x, again, n_tok=T, logits=lg)
                torch.cuda.synchronize()
                assert torch.equal(again, eager)
        finally:
            ctx.set_mode(0)
        got = eager.cpu().numpy()
        ref = oracle_tokens(L, xs, lg_h, [0, 47, 95])
        for t, (oo, _, _) in ref.items():
            rel = cases.rel_l2(got[t], oo)
            say("format groups, token %d: rel-L2 %.2e" % (t, rel))
            assert rel <= TOL_BF16
    finally:
        L.free()


def test_grouped_in_place_residual_update(torch_dev, ctx, layer):
    """x, residual and out the same buffer on the grouped path (router and
    RMSNorm on the device) equals the call with separate buffers."""
    torch = torch_dev
    T = 80
    nw = torch.from_numpy(cases.norm_w(61, 0)).cuda()
    desc = Q.MoeLayer.from_buffer_copy(layer.desc)
    desc.norm_w, desc.norm_eps = nw.data_ptr(), 1e-6
    h = torch.from_numpy(np.stack([cases.token_x(66, 2, t) for t in range(T)])).cuda()
    ref = torch.empty_like(h)
    ctx.set_mode(2)
    try:
        ctx.moe_forward(desc, h, ref, n_tok=T, residual=h)
        torch.cuda.synchronize()
        ctx.moe_forward(desc, h, h, n_tok=T, residual=h)
        torch.cuda.synchronize()
    finally:
        ctx.set_mode(0)
    assert torch.equal(h, ref)


@pytest.mark.parametrize("mix", ["iq2a", "iq2b"])
def test_grouped_iq_vs_per_token_kernels(torch_dev, ctx, mix):
    """IQ layers, all 64 tokens of a batch: grouped kernels against the fp32
    per-token kernels of the same library."""
    from qw6_amd.workload import SynthLayer
    L = SynthLayer(ctx, 73, 0, mix)
    try:
        T = 64
        lg = S.zipf_logits(74, T)
        xs = np.stack([cases.token_x(73, 6, t) for t in range(T)])
        out_g, idx_g, _ = run(torch_dev, ctx, L, xs, logits=lg, mode=2)
        out_p, idx_p, _ = run(torch_dev, ctx, L, xs, logits=lg, mode=1)
        assert np.array_equal(idx_g, idx_p)
        rels = [cases.rel_l2(out_g[t], out_p[t]) for t in range(T)]
        say("%s grouped vs per-token rel-L2 max %.2e mean %.2e" % (mix, max(rels), np.mean(rels)))
        assert max(rels) <= TOL_BF16
        assert np.mean(rels) <= TOL_MEAN
    finally:
        L.free()
