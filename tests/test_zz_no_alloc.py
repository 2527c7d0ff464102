"""qw6_hip_moe_forward_noalloc (the entry point that allocates nothing)
against qw6_hip_moe_forward, through the C ABI: bit-identical outputs and
selections (the same per-token kernels, in the same mode, on a different
workspace), on calls in a row, the last with a smaller input; device free
memory does not change across the calls."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import cases
import qw6_amd as Q

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_noalloc_matches_moe_forward():
    import torch
    from qw6_amd.workload import SynthLayer
    assert torch.cuda.is_available(), "no GPU visible"
    ctx = Q.Context(0, max_tokens=18)
    big = SynthLayer(ctx, 11, 0, "q4k")
    small = SynthLayer(ctx, 31, 0, "iq2m", hidden=1024, inter=256, n_experts=64, top_k=4)
    try:
        nw = torch.from_numpy(cases.norm_w(11, 0)).cuda()
        dbig = Q.MoeLayer.from_buffer_copy(big.desc)
        dbig.norm_w, dbig.norm_eps = nw.data_ptr(), 1e-6
        # (layer, hidden, tokens, residual, mode): both entry points run the
        # same per-token kernels in the same mode (the regular one would take
        # the grouped kernels for 17 tokens or more in mode 0). 8 tokens and 4
        # in mode 3 run the small-batch MFMA kernels (k_mx_*) on the static
        # array's operand regions, in two 4-token launches and in one; 18 in
        # mode 1 the fp32 kernels in launches of 16 and 2 tokens.
        calls = [(dbig, 2048, 3, True, 0), (dbig, 2048, 8, True, 3), (dbig, 2048, 4, True, 3),
                 (dbig, 2048, 18, True, 1), (dbig, 2048, 6, True, 0),
                 (small.desc, 1024, 1, False, 0)]
        # warm both paths once (first-use allocations of the regular path
        # and of the runtime happen here, not in the measured calls)
        for d, H, T, res, mode in calls:
            x = torch.zeros(T, H, dtype=torch.float32, device="cuda")
            o = torch.zeros_like(x)
            ctx.set_mode(mode)
            ctx.moe_forward(d, x, o, n_tok=T)
            ctx.moe_forward_noalloc(d, x, o, n_tok=T)
        ctx.set_mode(0)
        torch.cuda.synchronize()
        for i, (d, H, T, res, mode) in enumerate(calls):
            say("noalloc call %d: hidden %d, %d tokens, mode %d" % (i, H, T, mode))
            ctx.set_mode(mode)
            xs = np.stack([cases.token_x(300 + i, 1, t, hidden=H) for t in range(T)])
            x = torch.from_numpy(xs).cuda()
            r = x.clone() if res else None
            want = torch.zeros_like(x)
            wi = torch.zeros(T, 8, dtype=torch.int32, device="cuda")
            ww = torch.zeros(T, 8, dtype=torch.float32, device="cuda")
            ctx.moe_forward(d, x, want, n_tok=T, residual=r, idx=wi, w=ww)
            torch.cuda.synchronize()
            got = torch.zeros_like(x)
            gi = torch.zeros_like(wi)
            gw = torch.zeros_like(ww)
            torch.cuda.synchronize()
            free0 = torch.cuda.mem_get_info()[0]   # only the call below runs from here
            ctx.moe_forward_noalloc(d, x, got, n_tok=T, residual=r, idx=gi, w=gw)
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info()[0] == free0, i
            assert torch.equal(got, want), i
            assert torch.equal(gi, wi) and torch.equal(gw, ww), i
        ctx.set_mode(0)
        # the grouped path needs context workspace: refused
        ctx.set_mode(2)
        try:
            x = torch.zeros(1, 2048, dtype=torch.float32, device="cuda")
            with pytest.raises(Q.Qw6HipError, match="without allocation"):
                ctx.moe_forward_noalloc(dbig, x, torch.zeros_like(x), n_tok=1)
        finally:
            ctx.set_mode(0)
    finally:
        big.free()
        small.free()
        ctx.close()
