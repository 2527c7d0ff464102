"""Non-finite hidden states through the layer entry point, the router logits
computed on the device (no logits given), on every path a call can take.

qw6 rejects a hidden state holding NaN or Inf after each half of a layer
(qw6_check_nan_inf, qw6.c:2485-2488), so what a drop-in owes it is: the
same expert indices as qw6's CPU path (qw6_cpu_moe_route on the logits that
the router matvec gives, qw6.c:2226-2249, 2796-2827), a non-finite output
wherever qw6's is non-finite, and a finite token beside poisoned ones in the
same call unchanged. Tokens: NaN at one column, all NaN, +Inf at one column,
-Inf at one column, and finite tokens. A NaN column makes every logit NaN,
so qw6 picks index 0 in every round; an infinite column makes the logits
+-Inf (the sign of each router row's weight there), whatever the summation
order, so the selection is exact on every path.

Paths: the fp32 per-token kernels (mode 1) and the small-batch MFMA kernels
(mode 3) at T = 1-4, the automatic choice (mode 0) at T = 1-4, the fp32
kernels' launches of more tokens (6 and 16 in one launch, the router with
one grid row per token too; 18 = 16 + 2), the grouped MFMA kernels (mode 2) at T = 5 and
at 64 (the poisoned tokens among 59 finite ones); and the fused RMSNorm with
the residual added (the decode-step glue) at T = 1, 6 and 16 on the fp32
kernels and 5 on the grouped ones. Bars: indices bit-exact; gate weights NaN where the oracle's
are, within 2e-5 elsewhere; outputs finite exactly where the oracle's are,
the finite tokens within rel-L2 1e-5 (2e-3 for the grouped call of 64).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import cases
import oracle as O
import qw6_amd as Q

pytestmark = pytest.mark.gpu

EPS = 1e-6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def poisoned_tokens(seed):
    """(name, x) of the non-finite tokens, then two finite ones."""
    base = [cases.token_x(seed, 5, t) for t in range(6)]
    out = []
    x = base[0].copy(); x[7] = np.nan; out.append(("nan@7", x))
    out.append(("all-nan", np.full_like(base[1], np.nan)))
    x = base[2].copy(); x[100] = np.inf; out.append(("+inf@100", x))
    x = base[3].copy(); x[2047] = -np.inf; out.append(("-inf@2047", x))
    out.append(("finite0", base[4]))
    out.append(("finite1", base[5]))
    return out


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
    def __init__(self, L, seed):
        self.L = L
        toks = poisoned_tokens(seed)
        fill = [cases.token_x(seed, 6, t) for t in range(64)]
        self.names = [n for n, _ in toks] + ["fill%d" % i for i in range(len(fill))]
        self.xs = np.stack([x for _, x in toks] + fill).astype(np.float32)
        self.npois = 4
        router = L.router_host()
        self.nw = cases.norm_w(seed, 0)
        need = set()
        self.lg, self.lgn = [], []
        for x in self.xs:
            lg = O.matvec(0, router, L.n_experts, L.hidden, x)
            lgn = O.matvec(0, router, L.n_experts, L.hidden, O.rmsnorm(x, self.nw, EPS))
            self.lg.append(lg)
            self.lgn.append(lgn)
            need.update(int(i) for i in O.moe_route(lg, L.top_k)[0])
            need.update(int(i) for i in O.moe_route(lgn, L.top_k)[0])
        ex = [L.expert_host(e) if e in need else None for e in range(L.n_experts)]
        self.ol = O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, router, ex, L.shared_host())
        self._want = {}

    def want(self, t, glue):
        """The oracle's (out, idx, w) of token t; with glue, of x + the layer
        applied to rmsnorm(x) (the router reads the normalised input)."""
        key = (t, glue)
        if key not in self._want:
            x = self.xs[t]
            if glue:
                o, i, w = O.moe_layer(self.ol, O.rmsnorm(x, self.nw, EPS), nthreads=8)
                o = (x + o).astype(np.float32)
            else:
                o, i, w = O.moe_layer(self.ol, x, nthreads=8)
            self._want[key] = (o, i, w)
        return self._want[key]


@pytest.fixture(scope="module", params=[("q4k", 11), ("iq2m", 21)], ids=["q4k", "iq2m"])
def case(request, torch_dev, ctx):
    from qw6_amd.workload import SynthLayer
    mix, seed = request.param
    say("non-finite layer", mix, seed)
    L = SynthLayer(ctx, seed, 0, mix)
    try:
        yield Case(L, seed)
    finally:
        L.free()


def run(torch, ctx, c, toks, mode, glue):
    L = c.L
    T = len(toks)
    dx = torch.from_numpy(np.ascontiguousarray(c.xs[toks])).cuda()
    dout = torch.zeros(T, L.hidden, dtype=torch.float32, device="cuda")
    didx = torch.full((T, L.top_k), -1, dtype=torch.int32, device="cuda")
    dw = torch.zeros(T, L.top_k, dtype=torch.float32, device="cuda")
    desc, keep = L.desc, None
    if glue:
        keep = torch.from_numpy(c.nw).cuda()
        desc = Q.MoeLayer.from_buffer_copy(L.desc)
        desc.norm_w, desc.norm_eps = keep.data_ptr(), EPS
    ctx.set_mode(mode)
    try:
        ctx.moe_forward(desc, dx, dout, n_tok=T, residual=dx if glue else None, idx=didx, w=dw)
        torch.cuda.synchronize()
    finally:
        ctx.set_mode(0)
    return dout.cpu().numpy(), didx.cpu().numpy(), dw.cpu().numpy()


def check(c, toks, out, idx, w, tol, glue, where):
    for j, t in enumerate(toks):
        oo, oi, ow = c.want(t, glue)
        tag = "%s token %d (%s)" % (where, t, c.names[t])
        assert np.array_equal(idx[j], oi), (tag, idx[j], oi)
        assert np.array_equal(np.isnan(w[j]), np.isnan(ow)), (tag, w[j], ow)
        assert np.abs(np.nan_to_num(w[j]) - np.nan_to_num(ow)).max() <= 2e-5, tag
        fin = np.isfinite(oo)
        assert np.array_equal(np.isfinite(out[j]), fin), tag
        if t < c.npois:
            assert not fin.all(), tag   # a poisoned token stays visible to the check
        if fin.all():
            assert cases.rel_l2(out[j], oo) <= tol, tag


@pytest.mark.parametrize("mode", [1, 3, 0], ids=["fp32", "mfma", "auto"])
@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_nonfinite_tokens_per_token_paths(torch_dev, ctx, case, mode, T):
    c = case
    n = 6
    for t0 in range(0, n, T):
        toks = [(t0 + j) % n for j in range(T)]
        say("non-finite mode %d T=%d tokens %s" % (mode, T, [c.names[t] for t in toks]))
        out, idx, w = run(torch_dev, ctx, c, toks, mode, False)
        check(c, toks, out, idx, w, 1e-5, False, "mode %d T=%d" % (mode, T))


@pytest.mark.parametrize("T", [6, 16, 18])
def test_nonfinite_tokens_fp32_launches(torch_dev, ctx, case, T):
    c = case
    toks = list(range(T))
    say("non-finite fp32 kernels T=%d" % T)
    out, idx, w = run(torch_dev, ctx, c, toks, 1, False)
    check(c, toks, out, idx, w, 1e-5, False, "mode 1 T=%d" % T)


@pytest.mark.parametrize("T", [5, 64])
def test_nonfinite_tokens_grouped(torch_dev, ctx, case, T):
    c = case
    toks = list(range(T)) if T < 64 else [6 + i for i in range(30)] + list(range(6)) + \
        [36 + i for i in range(28)]
    say("non-finite grouped T=%d" % T)
    out, idx, w = run(torch_dev, ctx, c, toks, 2, False)
    check(c, toks, out, idx, w, 1e-5 if T < 64 else 2e-3, False, "grouped T=%d" % T)


@pytest.mark.parametrize("T,mode", [(1, 1), (6, 1), (16, 1), (5, 2)],
                         ids=["decode", "fp32-6", "fp32-16", "grouped"])
def test_nonfinite_tokens_with_norm_and_residual(torch_dev, ctx, case, T, mode):
    c = case
    n = 6 if T <= 6 else T
    for t0 in range(0, n, T):
        toks = [(t0 + j) % n for j in range(T)]
        say("non-finite glue mode %d T=%d tokens %s" % (mode, T, [c.names[t] for t in toks]))
        out, idx, w = run(torch_dev, ctx, c, toks, mode, True)
        check(c, toks, out, idx, w, 1e-5, True, "glue mode %d T=%d" % (mode, T))
