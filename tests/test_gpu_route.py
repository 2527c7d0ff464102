"""qw6's routing rules through the layer entry point (qw6_hip_moe_forward with
given router logits), on every path the call can take, against the oracle.

qw6_cpu_moe_route (qw6.c:2796-2827, reached from qw6.c:2247-2249) runs top_k
rounds of a strict '>' scan from best = index 0 and sets each winner to -inf:
ties go to the lowest index, a NaN at index 0 wins the first round, a NaN
elsewhere never wins, and once only -inf and NaN are left index 0 is picked
again (so one token may select expert 0 at several ranks). The vectors below
put each of those cases in one token of a 256-expert layer:
  - the committed routing vectors (random, many exact ties, the Vulkan
    self-test KAT qw6_vk.c:1898-1920, -inf at every third index, all equal,
    qw6.c:3400-3412's four logits padded with -inf);
  - the NaN vectors of cases.nan_route_cases padded with NaN, an all-NaN
    token, NaN at index 0 before random logits, NaNs scattered elsewhere;
  - an all -inf token, and three finite logits among -inf.

Paths: the fp32 per-token kernels (mode 1) and the small-batch MFMA kernels
(mode 3) at T = 1-4, the automatic choice at T = 1-4, the fp32 kernels'
launches of more tokens (6 and 16 in one launch, 18 = 16 + 2; the automatic
choice at 10), and the grouped MFMA kernels (mode 2) at T = 5 and 64, on a
Q4_K / Q6_K layer and on the IQ2_M
mix. Bars: indices bit-exact for every token; gate weights NaN where the
oracle's are and within 2e-5 elsewhere; outputs NaN exactly where the
oracle's are, and the finite ones within rel-L2 1e-5 (per-token kernels and
grouped calls under 64 tokens) or 2e-3 (grouped, 64 tokens).
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

TOL = {1: 1e-5, 3: 1e-5, 0: 1e-5}   # per-token paths, by mode
TOL_GROUPED_SMALL = 1e-5
TOL_GROUPED = 2e-3


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


class Case:
    """A layer with its tokens (x, logits) and the oracle's answer per token,
    computed once and reused by every path."""

    def __init__(self, L, seed):
        self.L = L
        vecs = cases.route_vectors()
        zl = S.zipf_logits(seed + 1, 64 - len(vecs))
        self.names = [n for n, _ in vecs] + ["zipf%d" % i for i in range(len(zl))]
        self.lg = np.concatenate([np.stack([v for _, v in vecs]), zl]).astype(np.float32)
        self.xs = np.stack([cases.token_x(seed, 9, t) for t in range(len(self.lg))])
        need = set()
        for lg in self.lg:
            need.update(int(i) for i in O.moe_route(lg, L.top_k)[0])
        ex = [L.expert_host(e) if e in need else None for e in range(L.n_experts)]
        ol = O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, None, ex, L.shared_host())
        self.want = [O.moe_layer(ol, self.xs[t], logits=self.lg[t], nthreads=8)
                     for t in range(len(self.lg))]


@pytest.fixture(scope="module", params=[("q4k", 11), ("iq2m", 21)], ids=["q4k", "iq2m"])
def case(request, torch_dev, ctx):
    from qw6_amd.workload import SynthLayer
    mix, seed = request.param
    say("route layer", mix, seed)
    L = SynthLayer(ctx, seed, 0, mix)
    try:
        yield Case(L, seed)
    finally:
        L.free()


def run(torch, ctx, L, xs, lg, mode):
    T = xs.shape[0]
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    dl = torch.from_numpy(np.ascontiguousarray(lg)).cuda()
    dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
    didx = torch.full((T, L.top_k), -1, dtype=torch.int32, device="cuda")
    dw = torch.zeros(T, L.top_k, dtype=torch.float32, device="cuda")
    ctx.set_mode(mode)
    try:
        ctx.moe_forward(L.desc, dx, dout, n_tok=T, logits=dl, idx=didx, w=dw)
        torch.cuda.synchronize()
    finally:
        ctx.set_mode(0)
    return dout.cpu().numpy(), didx.cpu().numpy(), dw.cpu().numpy()


def check(c, toks, out, idx, w, tol, where):
    for j, t in enumerate(toks):
        oo, oi, ow = c.want[t]
        tag = "%s token %d (%s)" % (where, t, c.names[t])
        assert np.array_equal(idx[j], oi), (tag, idx[j], oi)
        assert np.array_equal(np.isnan(w[j]), np.isnan(ow)), tag
        assert np.abs(np.nan_to_num(w[j]) - np.nan_to_num(ow)).max() <= 2e-5, tag
        nan_o = np.isnan(oo)
        assert np.array_equal(np.isnan(out[j]), nan_o), tag
        if not nan_o.all():
            assert np.isfinite(out[j][~nan_o]).all(), tag
            assert cases.rel_l2(out[j][~nan_o], oo[~nan_o]) <= tol, tag


@pytest.mark.parametrize("mode", [1, 3, 0], ids=["fp32", "mfma", "auto"])
@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_route_rules_per_token_paths(torch_dev, ctx, case, mode, T):
    c = case
    nv = len(cases.route_vectors())
    for t0 in range(0, nv, T):
        toks = [(t0 + j) % nv for j in range(T)]
        say("route mode %d T=%d tokens %s" % (mode, T, [c.names[t] for t in toks]))
        out, idx, w = run(torch_dev, ctx, c.L, c.xs[toks], c.lg[toks], mode)
        check(c, toks, out, idx, w, TOL[mode], "mode %d T=%d" % (mode, T))


@pytest.mark.parametrize("T,mode", [(6, 1), (16, 1), (18, 1), (10, 0)])
def test_route_rules_fp32_launches(torch_dev, ctx, case, T, mode):
    c = case
    nv = len(cases.route_vectors())
    toks = [nv - T // 2 + j for j in range(T)]   # the last route vectors, then Zipf tokens
    say("route mode %d T=%d" % (mode, T))
    out, idx, w = run(torch_dev, ctx, c.L, c.xs[toks], c.lg[toks], mode)
    check(c, toks, out, idx, w, 1e-5, "mode %d T=%d" % (mode, T))


@pytest.mark.parametrize("T", [5, 64])
def test_route_rules_grouped(torch_dev, ctx, case, T):
    c = case
    nv = len(cases.route_vectors())
    starts = range(0, nv, T) if T < 64 else [0]
    tol = TOL_GROUPED if T >= 64 else TOL_GROUPED_SMALL
    for t0 in starts:
        toks = [(t0 + j) % len(c.lg) for j in range(T)]
        say("route grouped T=%d from token %d" % (T, t0))
        out, idx, w = run(torch_dev, ctx, c.L, c.xs[toks], c.lg[toks], 2)
        check(c, toks, out, idx, w, tol, "grouped T=%d" % T)
