#!/usr/bin/env python3
"""Write tests/golden/golden.npz from qw6's own CPU path (oracle/_ref).

Run in a checkout next to the reference tree after `make -C oracle ref`:
    python3 tests/golden/make_golden.py
Inputs are not stored: every case is regenerated from its seed by
qw6_amd.synth (exact integer arithmetic). The file holds the reference's
outputs only (fp32 bit patterns, expert indices, softmax weights).
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import oracle as O  # noqa: E402
from qw6_amd import synth as S  # noqa: E402
import cases  # noqa: E402

FORMATS = [S.Q_Q4_K_M, S.Q_Q5_K, S.Q_Q6_K, S.Q_IQ2_XXS, S.Q_IQ2_S, S.Q_IQ3_S]
MV_SHAPES = [(3, 256), (16, 512), (8, 2048), (5, 1280)]


def mv_case(q, rows, cols, seed):
    w = S.quant_matrix(seed, S.stream_id(0, S.K_GATE, q), q, rows, cols)
    x = S.f32_normal(seed, S.stream_id(0, S.K_X, q), cols, 1.0)
    return w, x


def main():
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libqw6ref.so not built (make -C oracle ref)")
    g = {}
    # fp16 decode over all 65536 halves
    h = np.array([R.ref_fp16_to_f32(v) for v in range(65536)], np.float32)
    g["fp16_sha256"] = np.frombuffer(hashlib.sha256(h.tobytes()).digest(), np.uint8)
    # matvec per format and shape
    for q in FORMATS:
        for rows, cols in MV_SHAPES:
            w, x = mv_case(q, rows, cols, 3)
            g["mv_%d_%dx%d" % (q, rows, cols)] = O.ref_matvec(q, w, rows, cols, x)
        w = S.quant_matrix(5, S.stream_id(0, S.K_UP, q), q, 2, 512)
        g["deq_%d" % q] = np.stack([O.ref_dequant_row(q, w, 2, 512, r) for r in range(2)])
    # cfg0: Q4_K 512 x 2048, seed 1
    w = S.quant_matrix(1, S.stream_id(0, S.K_GATE), S.Q_Q4_K_M, 512, 2048)
    x = S.f32_normal(1, S.stream_id(0, S.K_X), 2048, 1.0)
    g["cfg0_y"] = O.ref_matvec(S.Q_Q4_K_M, w, 512, 2048, x)
    # routing
    for name, (lg, k) in cases.route_cases().items():
        idx, wt = O.ref_moe_route(lg, k)
        g[name + "_idx"], g[name + "_w"] = idx, wt
    # rmsnorm
    xr = S.f32_normal(7, S.stream_id(0, S.K_X, 99), 2048, 1.0)
    g["rms_out"] = O.ref_rmsnorm(xr, cases.norm_w(7, 0))
    # single layers
    for mix, seed, shared, sr in (("q4k", 11, True, False), ("q4k", 12, True, False),
                                  ("q4k", 13, False, False), ("iq2m", 21, True, False),
                                  ("iq2m", 22, True, False), ("q4k", 14, True, True),
                                  ("iq2m", 23, True, True)):
        L = cases.HostLayer(seed, 0, mix, shared=shared, shared_router=sr)
        x = cases.token_x(seed, 0)
        lg = cases.router_logits(L, x)
        idx, _ = O.moe_route(lg, 8)
        ol = L.oracle_layer(set(int(i) for i in idx))
        out, ridx, rw = O.ref_moe_layer(ol, x)
        key = "layer_%s_s%d%s%s" % (mix, seed, "" if shared else "_noshared", "_sr" if sr else "")
        g[key + "_out"], g[key + "_idx"], g[key + "_w"] = out, ridx, rw
    # stack: 3 layers x 2 steps, h <- h + MoE_l(RMSNorm(h, w_l))  (qw6.c:2475-2484)
    seed = 41
    layers = [cases.HostLayer(seed, l, "iq2m") for l in range(3)]
    for step in range(2):
        hcur = cases.token_x(seed, 100, step)
        for l, L in enumerate(layers):
            xn = O.ref_rmsnorm(hcur, cases.norm_w(seed, l))
            lg = cases.router_logits(L, xn)
            idx, _ = O.moe_route(lg, 8)
            ol = L.oracle_layer(set(int(i) for i in idx))
            out, ridx, _ = O.ref_moe_layer(ol, xn)
            hcur = (hcur + out).astype(np.float32)
            g["stack_s%d_l%d_idx" % (step, l)] = ridx
        g["stack_s%d_h" % step] = hcur
    # batched tokens with given Zipf logits (prefill-style), 4 tokens
    seed = 51
    L = cases.HostLayer(seed, 0, "q4k")
    lg = S.zipf_logits(seed, 4)
    for t in range(4):
        x = cases.token_x(seed, 0, t)
        idx, _ = O.moe_route(lg[t], 8)
        ol = L.oracle_layer(set(int(i) for i in idx))
        out, ridx, rw = O.ref_moe_layer(ol, x, logits=lg[t])
        g["prefill_t%d_out" % t], g["prefill_t%d_idx" % t], g["prefill_t%d_w" % t] = out, ridx, rw
    path = Path(__file__).with_name("golden.npz")
    np.savez_compressed(path, **g)
    print("wrote", path, len(g), "arrays", path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
