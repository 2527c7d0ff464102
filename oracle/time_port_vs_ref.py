"""Calibration of the CPU baseline (test infrastructure, run where the
reference tree is, never on the GPU host): single-token MoE layer steps of
the seeded Q4_K / Q6_K layer (hidden 2048, 256 experts top-8, inter 512,
shared expert) through qw6's own CPU path (oracle/_ref, qw6.c compiled
unmodified) and through the oracle port, one thread each, alternating, on
the same inputs; prints both medians and checks the outputs are bitwise
equal.

    python oracle/time_port_vs_ref.py [steps]
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "tests"))

import cases  # noqa: E402
import oracle as O  # noqa: E402


def main():
    steps = int(sys.argv[1]) if len(sys.argv) > 1 else 20
    if O.ref() is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref)")
    L = cases.HostLayer(11, 0, "q4k")
    xs = [cases.token_x(11, 0, t) for t in range(steps)]
    t_ref, t_port = [], []
    for x in xs:
        lg = cases.router_logits(L, x)
        idx, _ = O.moe_route(lg, L.top_k)
        layer = L.oracle_layer(set(int(i) for i in idx))
        t0 = time.perf_counter()
        r = O.ref_moe_layer(layer, x, want_route=False)
        t1 = time.perf_counter()
        p, _, _ = O.moe_layer(layer, x)
        t2 = time.perf_counter()
        t_ref.append(t1 - t0)
        t_port.append(t2 - t1)
        ro = r[0] if isinstance(r, tuple) else r
        assert np.array_equal(np.asarray(ro, np.float32).view(np.uint32), p.view(np.uint32))
    cpu = None
    with open("/proc/cpuinfo") as fh:
        for line in fh:
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    print("%d steps on %s (%d logical CPUs), one thread:" % (steps, cpu, os.cpu_count()))
    print("  qw6's build  %.1f us/layer (median)" % (1e6 * np.median(t_ref)))
    print("  oracle port  %.1f us/layer (median), outputs bitwise equal" % (1e6 * np.median(t_port)))


if __name__ == "__main__":
    main()
