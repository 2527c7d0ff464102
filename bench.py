#!/usr/bin/env python3
"""Benchmark of the MI355X routed-expert MoE FFN path (one GPU).

Headline workload (`value`): one MoE FFN decode step, batch 1, hidden 2048,
256 experts top-8, expert intermediate 512, Q4_K gate/up + Q6_K down, F32
router [256 x 2048], one shared expert of the same shapes; synthetic seeded
weights resident in HBM. A step is one token through one MoE layer (router
GEMV, softmax top-8, 8 experts + shared expert gate/up/SiLU/down,
gate-weighted combine). Steps cycle through a pool of independently seeded
layers (default 40 x ~522 MB) and inputs: the rows one pass over the pool
reads (40 x 20.5 MB of selected experts) exceed the 256 MB Infinity Cache
(MALL) three times over, so repeats come from HBM (with 16 layers, 328 MB,
part of them were served from the MALL). `value` is microseconds per MoE
layer of the HIP-graph-replayed kernels, inputs already in HBM.

`roofline` is for the dominant kernel (gate/up/SiLU over the 8 selected
experts + shared): algorithmic bytes per launch over its average duration,
measured with dispatch-timestamped HIP events on the launch stream.
`traffic` is the HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE
counter runs, each scaled by what the same counter reads for an elementwise
y = 2x kernel over 512 MiB (read from the committed summary; null when
absent).

`cpu_baseline` times the repository's C restatement of qw6's CPU path (the
oracle port, pinned bitwise to qw6's own build where the repository is built)
on a bounded sample of the headline workload on this host, single thread as
qw6 runs it, with its OpenMP build beside it. `cpu_baselines` holds the same
for every workload: the 512 x 2048 Q4_K matvec, the Q4_K and IQ2_M decode
layers, two-token steps, tokens of the 512-token batch (per token-expert
pair) and single-token steps of the 40-layer stack.

`secondary` (with --workload all, the default) adds:
  iq2m_decode   the same layer with IQ2_XXS gate/up and IQ3_S / IQ2_S down;
  stack         40 such layers, h <- h + MoE_l(RMSNorm(h, w_l)), 128 single-
                token steps: tokens/s and aggregate GB/s;
  prefill_T512  512 tokens with Zipf(1.1)-skewed router logits through the
                grouped bf16-MFMA kernels, Q4_K / Q6_K experts: us/layer,
                TFLOP/s, MFMA fraction, HBM GB/s;
  mtp_T2        two tokens (MTP draft verification) with the router GEMV, and
                small batches (3, 4, 8, 16 tokens) through the automatic path
                (--workload mtp: these alone);
  prefill_T512_iq2xxs_iq3s  the grouped kernels on an IQ layer (IQ2_XXS
                gate/up, IQ3_S down, Q4_K / Q6_K shared expert);
  output_head   the greedy next-token head: final RMSNorm, Q6_K [248320 x
                2048] vocabulary projection and argmax, us/token and HBM GB/s.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sys
import time

# The oracle's OpenMP threads sleep between parallel regions instead of
# spinning (the CPU-baseline leg alternates them with host work).
os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")

HERE = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
HIDDEN, INTER, N_EXPERTS, TOP_K = 2048, 512, 256, 8
# calls of this many tokens or more take the grouped kernels on a Q4_K / Q6_K
# layer in the automatic mode (qw6_hip_set_mode)
GROUPED_MIN_TOKENS = 17
TRAFFIC_FILE = os.path.join(HERE, "profiles", "moe_gate_up_q4k_decode_traffic.json")
# The headline's kernel instantiations in a trace or counter file (the
# one-token kernels of the Q4_K / Q6_K layer at hidden 2048, inter 512:
# router <8 float4 per lane, 2 waves per router row>, gate/up <format 0 =
# Q4_K, 64 units per row>, down <T = 1, format 2 = Q6_K, 16 units>), keyed by
# the names the bench line gives them. The default run dispatches them first;
# other workloads of the same run use other instantiations or come later.
HEADLINE_KERNELS = {"k_moe_router": "k_moe_router_w<8, 2, false>",
                    "k_moe_gate_up1": "k_moe_gate_up1<0, 64, false>",
                    "k_moe_down": "k_moe_down<1, 2, 16, false>"}


# --prefill-mix layer kinds and the formats they hold
PREFILL_FORMATS = {
    "q4k": "Q4_K gate/up, Q6_K down",
    "iq2a": "IQ2_XXS gate/up, IQ3_S down, Q4_K/Q6_K shared",
    "iq2m": "IQ2_XXS gate/up, IQ3_S (even experts) / IQ2_S (odd) down, Q4_K/Q6_K shared",
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--pool", type=int, default=40)
    ap.add_argument("--workload", default="all",
                    choices=["all", "q4k", "iq2m", "stack", "prefill", "mtp", "head", "floor",
                             "gguf"])
    ap.add_argument("--stack-steps", type=int, default=128)
    ap.add_argument("--prefill-tokens", type=int, default=512)
    ap.add_argument("--prefill-mix", default="q4k", choices=sorted(PREFILL_FORMATS),
                    help="with --workload prefill: the layer formats (q4k: Q4_K gate/up, Q6_K "
                         "down; iq2a: IQ2_XXS gate/up, IQ3_S down; iq2m: IQ2_XXS gate/up, "
                         "IQ3_S / IQ2_S downs by expert)")
    ap.add_argument("--no-small-batch", action="store_true",
                    help="with --workload prefill: time the prefill_T512 case only (no T=2 and "
                         "small-batch cases), for a kernel profile of that workload alone")
    ap.add_argument("--small-batch-sizes", default="3,4,8,16",
                    help="token counts of the small-batch rows beside the two-token case "
                         "(comma-separated; 'none' for the two-token case alone)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="CPU-baseline budget over all workloads (the oracle port, one thread "
                         "and OpenMP)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="eager launches only (for counter collection)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="first run y = 2x over MIB MiB 4 times (counter calibration: "
                         "MIB MiB read and written per launch)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc csv outputs (FETCH_SIZE, WRITE_SIZE) into the traffic summary")
    ap.add_argument("--summarize-trace", nargs="+", metavar="PATH",
                    help="TRACE_DIR BENCH_JSON [PLAIN_JSON]: split a rocprofv3 --kernel-trace "
                         "csv of a decode workload run into the run's phases (BENCH_JSON: the "
                         "line that run printed) and print per-kernel duration statistics for "
                         "each phase as markdown, beside the line of the same command run "
                         "without the profiler (PLAIN_JSON)")
    ap.add_argument("--summarize-counters", nargs="+", metavar="PMC_DIR",
                    help="print the mean per dispatch of every counter in these rocprofv3 --pmc "
                         "csv outputs for each k_moe_/k_pre_/k_head/k_argmax kernel as markdown (FETCH_SIZE and "
                         "WRITE_SIZE scaled by the --calib-copy copy kernel, when present)")
    ap.add_argument("--summarize-stats", nargs="+", metavar="TRACE_DIR",
                    help="print the k_ kernels' duration statistics of rocprofv3 --kernel-trace "
                         "--stats outputs as markdown")
    ap.add_argument("--command", default="", help="command line recorded in the summary")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---- counter summaries -----------------------------------------------------------

def _pmc_rows(d):
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit("no counter_collection.csv under %s" % d)
    rows = []
    for f in files:
        with open(f) as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _per_kernel(rows, counter):
    """Mean counter value per dispatch of each kernel name (KiB for *_SIZE)."""
    acc = {}
    for r in rows:
        if r.get("Counter_Name") != counter:
            continue
        name = r["Kernel_Name"]
        disp = r.get("Dispatch_Id") or r.get("Correlation_Id")
        acc.setdefault(name, {}).setdefault(disp, 0.0)
        acc[name][disp] += float(r["Counter_Value"])
    return {k: (sum(v.values()) / len(v), len(v)) for k, v in acc.items()}


def summarize_pmc(fetch_dir, write_dir, calib_mib, command):
    f = _per_kernel(_pmc_rows(fetch_dir), "FETCH_SIZE")
    w = _per_kernel(_pmc_rows(write_dir), "WRITE_SIZE")
    nbytes = calib_mib * 1024 * 1024

    def pick(d, key):
        ks = [k for k in d if key in k]
        if not ks:
            raise SystemExit("kernel %s not in counters: %s" % (key, list(d)))
        return max(ks, key=lambda k: d[k][1])

    ck_f = pick(f, "MulFunctor")
    ck_w = pick(w, "MulFunctor")
    fac_f = nbytes / (f[ck_f][0] * 1024.0)
    fac_w = nbytes / (w[ck_w][0] * 1024.0)
    gu_f = pick(f, HEADLINE_KERNELS["k_moe_gate_up1"])
    gu_w = pick(w, HEADLINE_KERNELS["k_moe_gate_up1"])
    fetch = f[gu_f][0] * 1024.0 * fac_f
    write = w[gu_w][0] * 1024.0 * fac_w
    out = {
        "kernel": "k_moe_gate_up1",
        "workload": "decode layer, batch 1, Q4_K gate/up + Q6_K down, F32 router, shared expert",
        "fetch_bytes_per_launch": round(fetch),
        "write_bytes_per_launch": round(write),
        "traffic_bytes_per_launch": round(fetch + write),
        "dispatches": [f[gu_f][1], w[gu_w][1]],
        "copy_kernel": {"bytes": nbytes, "fetch_KiB": f[ck_f][0], "write_KiB": w[ck_w][0],
                        "fetch_factor": fac_f, "write_factor": fac_w},
        "other_kernels_KiB": {k: [round(f[k][0], 1), round(w.get(k, (0.0, 0))[0], 1)]
                              for k in f if k not in (gu_f, ck_f) and
                              any(v in k for v in HEADLINE_KERNELS.values())},
        "command": command,
    }
    print(json.dumps(out, indent=1))


def _short_kernel(name):
    n = name.replace("void ", "").replace("(anonymous namespace)::", "").replace("qw6::", "")
    return n.split("(")[0]


def summarize_counters(dirs, calib_mib, command):
    """Mean value per dispatch of each counter, per kernel of the path."""
    rows = []
    for d in dirs:
        rows.extend(_pmc_rows(d))
    counters = sorted(set(r["Counter_Name"] for r in rows))
    table, calib = {}, {}
    for c in counters:
        for k, (v, n) in _per_kernel(rows, c).items():
            if "MulFunctor" in k:
                calib[c] = v
                continue
            if "k_moe_" not in k and "k_pre_" not in k and "k_head" not in k and "k_argmax" not in k:
                continue
            table.setdefault(_short_kernel(k), {})[c] = (v, n)
    nbytes = calib_mib * 1024 * 1024
    print("Command (repository root R):\n\n```\n%s\n```\n" % command)
    print("Mean per dispatch; the dispatches each mean is over in parentheses.\n")
    ks = sorted(table)
    print("| Counter | " + " | ".join("`%s`" % k for k in ks) + " |")
    print("|---|" + "---|" * len(ks))
    for c in counters:
        if c not in set().union(*[set(table[k]) for k in ks]):
            continue
        cells = []
        for k in ks:
            v = table[k].get(c)
            cells.append("" if v is None else "%.0f (%d)" % v)
        print("| %s | " % c + " | ".join(cells) + " |")
    for c, what in (("FETCH_SIZE", "read"), ("WRITE_SIZE", "written")):
        if c in calib and calib[c] > 0:
            fac = nbytes / (calib[c] * 1024.0)
            print("\n%s (KiB): the copy kernel that reads and writes %d MiB counts %.1f KiB "
                  "-> factor %.4f; HBM bytes %s per launch:" % (c, calib_mib, calib[c], fac, what))
            for k in sorted(table):
                if c in table[k]:
                    print("- `%s`: %.0f B" % (k, table[k][c][0] * 1024.0 * fac))


def summarize_stats(dirs, command):
    """Markdown table of the k_* kernels' durations in rocprofv3 --kernel-trace
    --stats outputs (one column group per trace directory, named by it)."""
    print("Command (repository root R):\n\n```\n%s\n```\n" % command)
    print("| Trace | Kernel | Dispatches | Avg us | Min us | Max us | Share of the trace's k_ kernel time |")
    print("|---|---|---|---|---|---|---|")
    for d in dirs:
        files = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
        if not files:
            raise SystemExit("no kernel_stats.csv under %s" % d)
        rows = []
        with open(files[0]) as fh:
            for r in csv.DictReader(fh):
                name = _short_kernel(r["Name"])
                if name.startswith("k_") and not name.startswith("k_synth"):
                    rows.append((name, int(r["Calls"]), float(r["TotalDurationNs"]),
                                 float(r["AverageNs"]), float(r["MinNs"]), float(r["MaxNs"])))
        tot = sum(x[2] for x in rows) or 1.0
        for name, calls, total, avg, mn, mx in sorted(rows, key=lambda x: -x[2]):
            print("| %s | `%s` | %d | %.2f | %.2f | %.2f | %.1f %% |"
                  % (os.path.basename(d.rstrip("/")), name, calls, avg / 1e3, mn / 1e3, mx / 1e3,
                     100.0 * total / tot))


def summarize_trace(trace_dir, bench_json, command, plain_json=None):
    """Per-kernel duration statistics of a decode run's kernel trace, split
    into the run's phases by dispatch order (bench_decode's dispatch_plan:
    every layer step dispatches each of the three kernels once, in order).
    Of each of the three kernels the instantiation dispatched first is taken
    (the run's first decode workload: the headline's, HEADLINE_KERNELS, in the
    default run), and of it the first dispatches the plan counts."""
    import numpy as np
    with open(bench_json) as fh:
        line = [l for l in fh if l.startswith("{")][-1]
    bj = json.loads(line)
    plan = bj["dispatch_plan"]
    files = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit("no kernel_trace.csv under %s" % trace_dir)
    bases = {v.split("<")[0] for v in HEADLINE_KERNELS.values()}
    per = {}
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"]
                if _short_kernel(name).split("<")[0] not in bases:
                    continue
                per.setdefault(name, []).append(
                    (int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    first = {}   # base kernel name -> its instantiation dispatched first
    for name, d in per.items():
        base = _short_kernel(name).split("<")[0]
        if base not in first or min(d)[0] < min(per[first[base]])[0]:
            first[base] = name
    per = {name: per[name] for name in first.values()}
    total = sum(n for _, n in plan)
    if len(per) != 3:
        raise SystemExit("expected the three decode kernels, found %s" % sorted(per))
    for name in per:   # the first workload's dispatches come first
        per[name] = sorted(per[name])[:total]
    order = sorted(per, key=lambda k: min(t for t, _ in per[k]))
    print("# Kernel durations of `%s` by phase (rocprofv3 kernel trace, %d dispatches per kernel)\n"
          % (bj["config"]["workload"], total))
    print("Command (repository root R):\n\n```\n%s\n```\n" % command)
    print("| Kernel | Phase | Dispatches | Avg ns | Median ns | p10 ns | p90 ns |")
    print("|---|---|---|---|---|---|---|")
    for name in order:
        d = sorted(per[name])
        if len(d) != total:
            raise SystemExit("%s: %d dispatches, the plan says %d" % (name, len(d), total))
        durs = np.array([x for _, x in d], dtype=np.float64)
        i = 0
        for phase, n in plan:
            seg = durs[i:i + n]
            i += n
            short = _short_kernel(name)
            print("| `%s` | %s | %d | %.0f | %.0f | %.0f | %.0f |" % (
                short, phase, n, seg.mean(), np.median(seg), np.percentile(seg, 10),
                np.percentile(seg, 90)))
    runs = [("the profiled run", bj)]
    if plain_json:
        with open(plain_json) as fh:
            runs.insert(0, ("the same command without the profiler",
                            json.loads([l for l in fh if l.startswith("{")][-1])))
    for what, j in runs:
        k = j["kernels"]
        print("\nBench line of %s (HIP events around each kernel of the `profile` phase):" % what)
        for kn in ("k_moe_router", "k_moe_gate_up1", "k_moe_down"):
            print("- `%s`: %.3f us, %d algorithmic bytes, %.1f GB/s" % (
                kn, k[kn]["us"], k[kn]["bytes"], k[kn]["GBps"]))
        sp = j.get("us_per_layer_spread") or {}
        print("- layer (graph replays): median %s us, p10 %s, p90 %s over %s replays of %s layers"
              % (sp.get("median"), sp.get("p10"), sp.get("p90"), sp.get("replays"),
                 sp.get("layers_per_replay")))
        print("- roofline: %s" % json.dumps(j["roofline"]))


# ---- shared helpers ---------------------------------------------------------------

def algorithmic_bytes(pool, sel, hidden=HIDDEN, inter=INTER):
    """Mean bytes per decode layer step split into router / gate_up / down from
    the experts each step actually selected (sel[j] for pool layer j)."""
    import numpy as np
    from qw6_amd import synth as S
    L0 = pool[0]
    sh_gu = sum(S.row_bytes(m[1], m[3]) * m[2] for m in L0.shared[:2])
    sh_dn = S.row_bytes(L0.shared[2][1], L0.shared[2][3]) * L0.shared[2][2]
    r_b = N_EXPERTS * hidden * 4 + hidden * 4 + N_EXPERTS * 4
    gu, dn = [], []
    for j, L in enumerate(pool):
        gub = sum(2 * S.row_bytes(L.quants[int(e)][0], hidden) * inter for e in sel[j])
        dnb = sum(S.row_bytes(L.quants[int(e)][2], inter) * hidden for e in sel[j])
        gu.append(gub + sh_gu + hidden * 4 + N_EXPERTS * 4 + (TOP_K + 1) * inter * 4)
        dn.append(dnb + sh_dn + (TOP_K + 1) * inter * 4 + hidden * 4)
    gu_b, d_b = float(np.mean(gu)), float(np.mean(dn))
    step_b = r_b + gu_b + d_b - N_EXPERTS * 4 - (TOP_K + 1) * inter * 4
    return r_b, gu_b, d_b, step_b


def hbm_roofline(nbytes, us):
    """Roofline of an HBM-bound call: the bytes it must read over its time."""
    gbps = nbytes / us / 1e3
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes": int(nbytes)}


def flop_roofline(flops, nbytes, us):
    """Roofline of a batched call: its FLOP rate against the lower of the bf16
    MFMA peak and arithmetic intensity x HBM peak."""
    tf = flops / (us * 1e-6) / 1e12
    roof = min(MFMA_BF16_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBPS / 1e3)
    return {"bound": "hbm" if roof < MFMA_BF16_PEAK_TFLOPS else "mfma", "achieved": round(tf, 2),
            "peak": round(roof, 1), "unit": "TFLOP/s", "frac": round(tf / roof, 4),
            "flops": int(flops), "bytes": int(nbytes)}


def capture_graph(torch, fn):
    """fn(stream) captured as one HIP graph on a side stream (after one eager
    call that makes first-use allocations); returns (graph, stream)."""
    g = torch.cuda.CUDAGraph()
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        fn(s2.cuda_stream)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s2):
            fn(s2.cuda_stream)
    torch.cuda.synchronize()
    return g, s2


def graph_time(torch, fn, reps):
    """Seconds per replay of fn() captured as one HIP graph."""
    g, _ = capture_graph(torch, fn)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps, g


def graph_replay_times(torch, fn, reps):
    """Seconds of each of `reps` back-to-back replays of fn() captured as one
    HIP graph, each bracketed by timing events on the replay stream."""
    g, s2 = capture_graph(torch, fn)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    with torch.cuda.stream(s2):
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        for e0, e1 in evs:
            e0.record()
            g.replay()
            e1.record()
    torch.cuda.synchronize()
    return [1e-3 * e0.elapsed_time(e1) for e0, e1 in evs]


def host_cpu():
    """Host CPU model (the lscpu 'Model name' line) and logical CPU count."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "nproc": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0))}


# ---- CPU baseline: the oracle port on the host's cores ---------------------------
# The port (oracle/qw6_oracle.c) restates qw6's CPU path in its own fp32
# expression order and is pinned bitwise to qw6's build in the container the
# repository is built in; the GPU host never loads qw6's build. Each figure is
# a median over a bounded sample of the same workload, single-threaded as qw6
# runs it, and again with the port's row-parallel OpenMP build (bitwise the
# same outputs).

CPU_THREADS_MAX = 16   # the host CPU share of one GPU on the machines this runs on


def _cpu_threads():
    return max(1, min(CPU_THREADS_MAX, len(os.sched_getaffinity(0))))


def _timed(fn, budget_s, nmax, nmin=2):
    """Durations (s) returned by fn(i) for i = 0, 1, ... until the budget or
    nmax calls are spent (at least nmin calls)."""
    ts = []
    t_end = time.perf_counter() + budget_s
    while (len(ts) < nmax and time.perf_counter() < t_end) or len(ts) < nmin:
        ts.append(fn(len(ts)))
    return ts


class PortLayer:
    """Host copies of one device layer for the oracle: router and shared
    expert at once, routed experts copied on first use (never timed)."""

    def __init__(self, L, norm_w=None):
        import oracle as O
        self.O, self.L = O, L
        self.router = L.router_host() if L.router is not None else None
        self.shared = L.shared_host()
        self.norm_w = norm_w
        self.cache = {}

    def layer(self, logits):
        O, L = self.O, self.L
        idx, _ = O.moe_route(logits, L.top_k)
        for e in set(int(i) for i in idx):
            if e not in self.cache:
                self.cache[e] = L.expert_host(e)
        ex = [self.cache.get(e) for e in range(L.n_experts)]
        return O.Layer(L.hidden, L.inter, L.n_experts, L.top_k, self.router, ex, self.shared)

    def step(self, x, logits=None, nthreads=1):
        """One token through the layer on the CPU: (output, seconds). The
        router GEMV (when no logits are given), routing, the expert matvecs,
        SiLU and the combine are timed; copying the selected experts to the
        host beforehand is not."""
        O = self.O
        lg = logits if logits is not None else O.matvec(0, self.router, self.L.n_experts,
                                                         self.L.hidden, x, nthreads=nthreads)
        layer = self.layer(lg)
        t0 = time.perf_counter()
        out, _, _ = O.moe_layer(layer, x, logits=logits, nthreads=nthreads)
        return out, time.perf_counter() - t0


def _cpu_entry(unit, single, multi, nt, sample, scale=1.0, extra=None):
    import numpy as np
    e = {"value": round(scale * 1e6 * float(np.median(single)), 1), "unit": unit, "cores": 1,
         "kind": "port", "sample": sample,
         "multicore": {"value": round(scale * 1e6 * float(np.median(multi)), 1), "cores": nt,
                       "kind": "port",
                       "sample": "%d of the same, OpenMP over %d threads" % (len(multi), nt)}}
    if extra:
        e.update(extra)
    return e


def cpu_matvec(budget_s):
    """One 512 x 2048 Q4_K dequant-matvec (the seeded matrix of the golden
    fixture) on the CPU."""
    sys.path.insert(0, HERE)
    import oracle as O
    from qw6_amd import synth as S
    w = S.quant_matrix(1, S.stream_id(0, S.K_GATE), S.Q_Q4_K_M, 512, 2048)
    x = S.f32_normal(1, S.stream_id(0, S.K_X), 2048, 1.0)
    nt = _cpu_threads()

    def run(nthreads):
        def f(_):
            t0 = time.perf_counter()
            O.matvec(S.Q_Q4_K_M, w, 512, 2048, x, nthreads=nthreads)
            return time.perf_counter() - t0
        return f
    single = _timed(run(1), budget_s * 0.6, 2000, 20)
    multi = _timed(run(nt), budget_s * 0.4, 2000, 20)
    return _cpu_entry("us/matvec", single, multi, nt,
                      "%d calls (median), Q4_K W[512 x 2048] x fp32 x[2048], one thread" % len(single))


def cpu_decode_layer(L, xs_host, budget_s, what):
    """Single-token MoE layer steps (router GEMV, top-8, experts, combine) on
    the CPU through layer L, inputs xs_host in turn."""
    pl = PortLayer(L)
    nt = _cpu_threads()
    single = _timed(lambda i: pl.step(xs_host[i % len(xs_host)])[1], budget_s * 0.7, 200, 3)
    multi = _timed(lambda i: pl.step(xs_host[i % len(xs_host)], nthreads=nt)[1],
                   budget_s * 0.3, 100, 3)
    return _cpu_entry("us/layer", single, multi, nt,
                      "%d single-token %s layer steps (median), one pool layer, one thread"
                      % (len(single), what))


def cpu_two_tokens(L, xs_host, budget_s):
    """Two tokens (MTP draft verification) through layer L on the CPU: qw6
    runs them one after the other."""
    pl = PortLayer(L)
    nt = _cpu_threads()

    def pair(nthreads):
        def f(i):
            a = xs_host[(2 * i) % len(xs_host)]
            b = xs_host[(2 * i + 1) % len(xs_host)]
            return pl.step(a, nthreads=nthreads)[1] + pl.step(b, nthreads=nthreads)[1]
        return f
    single = _timed(pair(1), budget_s * 0.7, 100, 2)
    multi = _timed(pair(nt), budget_s * 0.3, 50, 2)
    return _cpu_entry("us/layer", single, multi, nt,
                      "%d two-token steps (median) with the router GEMV, one thread" % len(single))


def cpu_prefill_tokens(L, xs_host, lg_host, budget_s, T):
    """Tokens of a T-token batch with given router logits through layer L on
    the CPU (qw6 runs a batch token by token): microseconds per token-expert
    pair (top_k routed + the shared expert per token), and per token and per
    T-token layer beside it."""
    pl = PortLayer(L)
    nt = _cpu_threads()
    n = len(xs_host)
    pairs = L.top_k + (1 if L.shared is not None else 0)
    single = _timed(lambda i: pl.step(xs_host[i % n], lg_host[i % n])[1], budget_s * 0.7, n, 3)
    multi = _timed(lambda i: pl.step(xs_host[i % n], lg_host[i % n], nthreads=nt)[1],
                   budget_s * 0.3, n, 3)
    import numpy as np
    tok_us = 1e6 * float(np.median(single))
    return _cpu_entry("us/token-expert pair", single, multi, nt,
                      "%d tokens of the %d-token batch (median), given Zipf logits, one thread; "
                      "%d token-expert pairs per token" % (len(single), T, pairs),
                      scale=1.0 / pairs,
                      extra={"us_per_token": round(tok_us, 1),
                             "us_per_layer_T%d" % T: round(T * tok_us, 1)})


def cpu_stack_token(stk, xs_host, budget_s):
    """Single-token steps of the whole stack on the CPU: h <- h + MoE_l(
    RMSNorm(h, w_l)) for every layer (qw6.c:2475-2484), RMSNorm and the
    residual add timed with the layers."""
    sys.path.insert(0, HERE)
    import numpy as np
    import oracle as O
    nw = stk.norm_w.cpu().numpy()
    pls = [PortLayer(L) for L in stk.layers]
    nt = _cpu_threads()

    def token(nthreads):
        def f(i):
            h = np.array(xs_host[i % len(xs_host)], np.float32)
            tot = 0.0
            for l, pl in enumerate(pls):
                t0 = time.perf_counter()
                xn = O.rmsnorm(h, nw[l], stk.eps)
                tot += time.perf_counter() - t0
                out, dt = pl.step(xn, nthreads=nthreads)
                t0 = time.perf_counter()
                h = (h + out).astype(np.float32)
                tot += dt + time.perf_counter() - t0
            return tot
        return f
    single = _timed(token(1), budget_s * 0.7, 8, 1)
    multi = _timed(token(nt), budget_s * 0.3, 8, 1)
    return _cpu_entry("us/token", single, multi, nt,
                      "%d single-token steps through all %d layers (median), one thread"
                      % (len(single), len(pls)))


# ---- workloads --------------------------------------------------------------------

def bench_decode(torch, Q, S, ctx, pool, X, out, idx, args, profile=True):
    import numpy as np
    P = len(pool)

    def step(k, sp):
        j = k % P
        ctx.moe_forward(pool[j].desc, X[j], out[j], n_tok=1, idx=idx[j], stream=sp)

    sp = torch.cuda.current_stream().cuda_stream
    for k in range(args.warmup):
        step(k, sp)
    torch.cuda.synchronize()
    r_b, gu_b, d_b, step_b = algorithmic_bytes(pool, idx.cpu().numpy())

    K = args.steps
    t0 = time.perf_counter()
    for k in range(K):
        step(k, sp)
    torch.cuda.synchronize()
    eager_us = 1e6 * (time.perf_counter() - t0) / K
    if args.no_graph:
        us_layer, steps, spread = eager_us, K, None
    else:
        # the K timed steps (layer k % P for step k) captured as one graph;
        # 20 replays of it, each timed on its own: the median, p10 and p90 of
        # the per-layer time over the replays
        reps = 20
        per = np.array(graph_replay_times(torch, lambda s: [step(k, s) for k in range(K)], reps))
        per_layer = 1e6 * per / K
        us_layer, steps = float(np.median(per_layer)), K
        spread = {"replays": reps, "layers_per_replay": K,
                  "median": round(us_layer, 3),
                  "p10": round(float(np.percentile(per_layer, 10)), 3),
                  "p90": round(float(np.percentile(per_layer, 90)), 3),
                  "min": round(float(per_layer.min()), 3)}
    res = {"us_per_layer": round(us_layer, 3), "eager_us_per_layer": round(eager_us, 3),
           "steps": steps, "bytes_per_step": int(step_b),
           "hbm_GBps": round(step_b / us_layer / 1e3, 1),
           "hbm_frac": round(step_b / us_layer / 1e3 / HBM_PEAK_GBPS, 4),
           "us_per_layer_spread": spread}
    if profile:
        # per-kernel durations from each kernel's own dispatch timestamps (HIP
        # events recorded by hipExtLaunchKernel on the launch stream)
        nprof = min(K, 256)
        ctx.profile(nprof)
        for k in range(nprof):
            step(k, sp)
        ms, calls = ctx.profile_read()
        ctx.profile(0)
        kus = [1e3 * m / calls for m in ms]
        res["kernels"] = {
            "k_moe_router": {"us": round(kus[0], 3), "bytes": int(r_b),
                             "GBps": round(r_b / kus[0] / 1e3, 1)},
            "k_moe_gate_up1": {"us": round(kus[1], 3), "bytes": int(gu_b),
                              "GBps": round(gu_b / kus[1] / 1e3, 1)},
            "k_moe_down": {"us": round(kus[2], 3), "bytes": int(d_b),
                           "GBps": round(d_b / kus[2] / 1e3, 1)},
        }
        res["profiled_calls"] = calls
    # the order in which this function dispatched layer steps (each step one
    # launch of each of the three kernels), for splitting a kernel trace
    plan = [("warmup", args.warmup), ("eager", K)]
    if not args.no_graph:
        plan += [("capture-call", K), ("replay-warmup", 2 * K), ("timed-replays", 20 * K)]
    if profile:
        plan.append(("profile", nprof))
    res["dispatch_plan"] = plan
    return res


def bench_gguf(torch, Q, S, ctx, pool, X, out, idx):
    """A cfg1-shaped layer written as a GGUF file, made resident by the
    library's loader (qw6_hip_gguf_moe_layer: parse, bind, stream through
    pinned staging), then run: load GB/s (file in the page cache) and the
    loaded layer's decode us/layer beside the synthetic layer's."""
    import tempfile
    import numpy as np
    from qw6_amd import gguf as G
    L = pool[0]
    packs = []
    for k in range(3):
        q = L.quants[0][k]
        packs.append((q, [L.expert_host(e)[k][0] for e in range(L.n_experts)]))
    ts = G.moe_layer_tensors(0, L.hidden, L.inter, L.router_host(), packs, shared=L.shared_host())
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "layer.gguf")
        G.write_gguf(path, [("general.architecture", G.T_STR, "qwen35moe")], ts)
        size = os.path.getsize(path)
        with G.GgufFile(path) as f:
            t0 = time.perf_counter()
            desc, E = f.moe_layer(ctx, 0)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
    try:
        o_file = torch.zeros_like(out[0])
        i_file = torch.zeros_like(idx[0])
        ctx.moe_forward(desc, X[0], o_file, n_tok=1, idx=i_file)
        ctx.moe_forward(L.desc, X[0], out[0], n_tok=1, idx=idx[0])
        torch.cuda.synchronize()
        same = bool(torch.equal(o_file, out[0]) and torch.equal(i_file, idx[0]))
        sec, _ = graph_time(torch, lambda s: [ctx.moe_forward(desc, X[0], o_file, n_tok=1, idx=i_file,
                                                               stream=s) for _ in range(16)], 20)
    finally:
        E.free()
    return {"file_MB": round(size / 1e6, 1), "load_s": round(dt, 4),
            "load_GBps": round(size / dt / 1e9, 2), "decode_us_per_layer": round(1e6 * sec / 16, 3),
            "bit_identical_to_synthetic_layer": same,
            "workload": "one cfg1 layer (256 Q4_K/Q6_K experts + shared) written to a GGUF file "
                        "and loaded; the same layer replayed 16 times per graph (MALL-resident)"}


def bench_floor(torch, Q, ctx):
    """The cost of one dependent kernel in a replayed graph: 24 argmax calls
    over 1024 floats (a one-block partial pass and a one-block final pass,
    each one memory round trip) captured back to back, so 48 tiny kernels
    each wait for the one before. A decode layer is three dependent kernels."""
    x = torch.randn(1024, dtype=torch.float32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    n = 24
    sec, _ = graph_time(torch, lambda s: [ctx.argmax(x, 1024, out, s) for _ in range(n)], 50)
    per_kernel = 1e6 * sec / (2 * n)
    return {"us_per_dependent_kernel": round(per_kernel, 3),
            "three_kernel_chain_us": round(3 * per_kernel, 3)}


VOCAB = 248320


def bench_head(torch, Q, S, ctx, args):
    """The greedy output head: final RMSNorm, Q6_K [248320 x 2048] vocabulary
    projection (417 MB streamed per token) and argmax, per token."""
    q = S.Q_Q6_K
    rb = S.row_bytes(q, HIDDEN)
    P = 2   # two resident heads, alternated, so no replay reads the same weights twice in a row
    ws = []
    for j in range(P):
        w = torch.empty(VOCAB * rb, dtype=torch.uint8, device="cuda")
        Q.synth_blocks(w, q, VOCAB * HIDDEN // 256, 5000 + j, S.stream_id(0, S.K_OUTPUT))
        ws.append(w)
    x = torch.empty(P, HIDDEN, dtype=torch.float32, device="cuda")
    nw = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    for j in range(P):
        Q.synth_normal(x[j], HIDDEN, 1.0, 5010 + j, S.stream_id(0, S.K_X))
    Q.synth_normal(nw, HIDDEN, 0.1, 5020, S.stream_id(0, S.K_ONORM), mean=1.0)
    lg = torch.empty(P, VOCAB, dtype=torch.float32, device="cuda")
    tok = torch.zeros(P, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()

    def fwd(sp):
        for j in range(P):
            ctx.output_greedy((ws[j].data_ptr(), q, VOCAB, HIDDEN), x[j], lg[j], tok[j:j + 1],
                              norm_w=nw, stream=sp)
    sec, _ = graph_time(torch, fwd, 20)
    us = 1e6 * sec / P
    nbytes = VOCAB * rb + 2 * HIDDEN * 4 + VOCAB * 4   # weights, x and norm weight, logits
    res = {"us_per_token": round(us, 2), "bytes": nbytes, "hbm_GBps": round(nbytes / us / 1e3, 1),
           "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4),
           "workload": "output head: RMSNorm + Q6_K [248320 x 2048] projection + greedy argmax, "
                       "one token, two resident heads alternated"}
    ws.clear()
    return res


def bench_stack(torch, Q, S, ctx, args, cpu=None):
    """40 IQ2_M-mix layers, h <- h + MoE_l(RMSNorm(h, w_l)), single-token steps
    (qw6_amd.workload.SynthStack: the norm fused into each layer's call, the
    hidden state updated in place, the step captured as one HIP graph)."""
    from qw6_amd.workload import SynthStack
    NL, NS = 40, args.stack_steps
    log("stack: building %d layers" % NL)
    stk = SynthStack(ctx, 3000, NL, "iq2m")
    X = torch.empty(NS, HIDDEN, dtype=torch.float32, device="cuda")
    for s in range(NS):
        Q.synth_normal(X[s], HIDDEN, 1.0, 3001, S.stream_id(s, S.K_X))
    h = torch.empty(1, HIDDEN, dtype=torch.float32, device="cuda")
    h.copy_(X[0])
    idx = torch.zeros(NL, TOP_K, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    # the step is captured once; each token's input is copied in before its replay
    g = stk.capture(h, idx)
    for s in range(4):
        h.copy_(X[s])
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(NS):
        h.copy_(X[s])
        g.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    r_b, gu_b, d_b, step_b = algorithmic_bytes(stk.layers, idx.cpu().numpy())
    tok_bytes = step_b * NL
    res = {"layers": NL, "steps": NS, "tokens_per_s": round(NS / wall, 1),
           "us_per_token": round(1e6 * wall / NS, 2),
           "us_per_layer": round(1e6 * wall / NS / NL, 3),
           "bytes_per_token": int(tok_bytes),
           "hbm_GBps": round(tok_bytes * NS / wall / 1e9, 1),
           "resident_GB": round(stk.resident_bytes() / 1e9, 2),
           "workload": "40 layers IQ2_XXS gate/up + IQ3_S/IQ2_S down, F32 router, shared "
                       "expert, RMSNorm (eps 1e-6) fused before each layer, residual in "
                       "place; 128 single-token steps with fresh inputs"}
    if cpu is not None:
        cpu["stack_40_layers_token"] = cpu_stack_token(stk, X[:8].cpu().numpy(),
                                                       args.cpu_seconds * 0.3)
    stk.free()
    return res


def bench_prefill(torch, Q, S, ctx, pool, args, with_t2=True,
                  formats=PREFILL_FORMATS["q4k"], cpu=None, with_grouped=True):
    """T tokens with Zipf-skewed logits through the grouped MFMA kernels
    (with_grouped), plus (with_t2) the T=2 MTP case through the per-token
    kernels with the router GEMV and the small-batch rows."""
    import numpy as np
    if not with_grouped:
        return None, bench_mtp(torch, Q, S, ctx, pool, args)
    T = args.prefill_tokens
    P = min(2, len(pool))
    lg_h = [S.zipf_logits(4000 + j, T) for j in range(P)]
    lg = [torch.from_numpy(a).cuda() for a in lg_h]
    X = torch.empty(P, T, HIDDEN, dtype=torch.float32, device="cuda")
    for j in range(P):
        Q.synth_normal(X[j], T * HIDDEN, 1.0, 4001, S.stream_id(j, S.K_X))
    out = torch.empty(P, T, HIDDEN, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.set_mode(2)
    try:
        def fwd(sp):
            for j in range(P):
                ctx.moe_forward(pool[j].desc, X[j], out[j], n_tok=T, logits=lg[j], stream=sp)
        fwd(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        reps = 10
        sec, _ = graph_time(torch, fwd, reps)
    finally:
        ctx.set_mode(0)
    us = 1e6 * sec / P
    flops, byts = [], []
    L0 = pool[0]
    for j in range(P):
        top = np.argsort(-lg_h[j], axis=1, kind="stable")[:, :TOP_K]
        used = np.unique(top)
        n_ent = T * TOP_K + T
        flops.append(2.0 * n_ent * 3 * HIDDEN * INTER)
        byts.append(sum(pool[j].expert_bytes(int(e)) for e in used) + L0.shared_bytes()
                    + 2 * T * HIDDEN * 4 + T * N_EXPERTS * 4)
    fl, by = float(np.mean(flops)), float(np.mean(byts))
    tf = fl / (us * 1e-6) / 1e12
    ai = fl / by
    roof = min(MFMA_BF16_PEAK_TFLOPS, ai * HBM_PEAK_GBPS / 1e3)
    res = {"tokens": T, "us_per_layer": round(us, 2), "TFLOPs": round(tf, 2),
           "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
           "roofline_TFLOPs": round(roof, 1), "roofline_frac": round(tf / roof, 4),
           "flops": int(fl), "bytes": int(by), "hbm_GBps": round(by / us / 1e3, 1),
           "tokens_per_s": round(T / (us * 1e-6), 1),
           "workload": "T=%d, hidden 2048, 256 experts top-8 + shared, %s; router logits "
                       "given, Zipf(1.1)-skewed (Gumbel-top-k)" % (T, formats)}
    if cpu is not None:   # a sample of the batch's tokens through the CPU port
        n = min(T, 64)
        cpu["prefill_T%d_pair" % T] = cpu_prefill_tokens(L0, X[0, :n].cpu().numpy(), lg_h[0][:n],
                                                         args.cpu_seconds * 0.15, T)
    if not with_t2:
        return res, None
    return res, bench_mtp(torch, Q, S, ctx, pool, args)


def bench_mtp(torch, Q, S, ctx, pool, args):
    """T = 2 (MTP draft verification) through the per-token kernels with the
    router GEMV, then the small-batch rows (--small-batch-sizes)."""
    import numpy as np
    X2 = torch.empty(len(pool), 2, HIDDEN, dtype=torch.float32, device="cuda")
    for j in range(len(pool)):
        Q.synth_normal(X2[j], 2 * HIDDEN, 1.0, 4002, S.stream_id(j, S.K_X))
    o2 = torch.empty_like(X2)
    i2 = torch.zeros(len(pool), 2, TOP_K, dtype=torch.int32, device="cuda")

    def fwd2(sp):
        for j in range(len(pool)):
            ctx.moe_forward(pool[j].desc, X2[j], o2[j], n_tok=2, idx=i2[j], stream=sp)
    # at least 10 replays of the pool (16 layers each), whatever --steps is
    sec2, _ = graph_time(torch, fwd2, max(10, args.steps // len(pool)))
    us2 = 1e6 * sec2 / len(pool)
    sel = i2.cpu().numpy()
    b2 = []
    for j, L in enumerate(pool):
        used = np.unique(sel[j])
        b2.append(sum(L.expert_bytes(int(e)) for e in used) + L.shared_bytes()
                  + N_EXPERTS * HIDDEN * 4 + 4 * HIDDEN * 4)
    b2m = float(np.mean(b2))
    res_t2 = {"tokens": 2, "us_per_layer": round(us2, 3), "bytes": int(b2m),
              "hbm_GBps": round(b2m / us2 / 1e3, 1),
              "distinct_experts_mean": round(float(np.mean([len(np.unique(s)) for s in sel])), 2),
              "roofline": hbm_roofline(b2m, us2),
              "workload": "T=2 through the per-token fp32 kernels with the router GEMV, "
                          "Q4_K/Q6_K layer pool"}
    # small batches through the automatic path: up to 16 tokens take the
    # fp32 per-token kernels (one grid row per token) on this layer
    small, small_roof = {}, {}
    sizes = [] if args.small_batch_sizes in ("", "none") else \
        [int(v) for v in args.small_batch_sizes.split(",")]
    for Ts in sizes:
        Xs = torch.empty(len(pool), Ts, HIDDEN, dtype=torch.float32, device="cuda")
        for j in range(len(pool)):
            Q.synth_normal(Xs[j], Ts * HIDDEN, 1.0, 4010 + Ts, S.stream_id(j, S.K_X))
        os_ = torch.empty_like(Xs)
        is_ = torch.zeros(len(pool), Ts, TOP_K, dtype=torch.int32, device="cuda")

        def fwds(sp, Ts=Ts, Xs=Xs, os_=os_, is_=is_):
            for j in range(len(pool)):
                ctx.moe_forward(pool[j].desc, Xs[j], os_[j], n_tok=Ts, idx=is_[j], stream=sp)
        secs, _ = graph_time(torch, fwds, max(10, args.steps // len(pool)))
        us_s = 1e6 * secs / len(pool)
        small["T%d" % Ts] = round(us_s, 3)
        # bytes one call must read: the distinct selected experts' matrices,
        # the shared expert, the router and the inputs (calls that take the
        # grouped kernels: the lower of the HBM and MFMA roofs)
        ss = is_.cpu().numpy()
        bs = float(np.mean([sum(L.expert_bytes(int(e)) for e in np.unique(ss[j])) + L.shared_bytes()
                            + N_EXPERTS * HIDDEN * 4 + 2 * Ts * HIDDEN * 4
                            for j, L in enumerate(pool)]))
        if Ts >= GROUPED_MIN_TOKENS:
            fl = 2.0 * (Ts * TOP_K + Ts) * 3 * HIDDEN * INTER
            small_roof["T%d" % Ts] = flop_roofline(fl, bs, us_s)
        else:
            small_roof["T%d" % Ts] = hbm_roofline(bs, us_s)
    res_t2["small_batch_us_per_layer"] = small
    res_t2["small_batch_roofline"] = small_roof
    return res_t2


def main():
    args = parse()
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], args.calib_copy or 512,
                      args.command)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters, args.calib_copy or 512, args.command)
        return
    if args.summarize_stats:
        summarize_stats(args.summarize_stats, args.command)
        return
    if args.summarize_trace:
        st = args.summarize_trace
        if len(st) not in (2, 3):
            raise SystemExit("--summarize-trace takes TRACE_DIR BENCH_JSON [PLAIN_JSON]")
        summarize_trace(st[0], st[1], args.command, st[2] if len(st) == 3 else None)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: the MoE FFN path is benchmarked on a single "
              "MI355X; --gpus %d is not run (sharding is a design note, not a benchmark)."
              % args.gpus, file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import qw6_amd as Q
    from qw6_amd import synth as S
    from qw6_amd.workload import SynthLayer

    torch.cuda.set_device(0)
    if args.calib_copy:
        n = args.calib_copy * 1024 * 1024 // 4
        a = torch.ones(n, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(4):   # reads MIB MiB, writes MIB MiB per launch
            torch.mul(a, 2.0, out=b)
        torch.cuda.synchronize()
        del a, b
    want_prefill = args.workload in ("all", "prefill", "mtp")
    cpu_cfg = None if args.no_cpu else {}
    ctx = Q.Context(0, max_tokens=max(args.prefill_tokens, 16) if want_prefill else 4)
    P = args.pool
    mix = ("iq2m" if args.workload == "iq2m" else
           args.prefill_mix if args.workload == "prefill" else "q4k")
    secondary = {}
    res_main = None
    pool = []
    if args.workload in ("all", "q4k", "iq2m", "prefill", "mtp", "gguf"):
        if args.workload == "prefill":
            P = 2   # the prefill figure alternates two layers
        log("building %d synthetic layers (%s)" % (P, mix))
        pool = [SynthLayer(ctx, 1000 + i, i, mix) for i in range(P)]
        X = torch.empty(P, HIDDEN, dtype=torch.float32, device="cuda")
        for i in range(P):
            Q.synth_normal(X[i], HIDDEN, 1.0, 77, S.stream_id(i, S.K_X))
        out = torch.empty(P, HIDDEN, dtype=torch.float32, device="cuda")
        idx = torch.zeros(P, TOP_K, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        if args.workload not in ("prefill", "mtp"):
            res_main = bench_decode(torch, Q, S, ctx, pool, X, out, idx, args)
            log("decode %s: %s" % (mix, json.dumps(res_main)))
    if want_prefill:
        pf, t2 = bench_prefill(torch, Q, S, ctx, pool, args,
                               with_t2=not args.no_small_batch and mix == "q4k",
                               formats=PREFILL_FORMATS[mix],
                               cpu=cpu_cfg if mix == "q4k" else None,
                               with_grouped=args.workload != "mtp")
        if pf is not None:
            secondary["prefill_T%d%s" % (args.prefill_tokens, "" if mix == "q4k" else "_" + mix)] = pf
            log("prefill: %s" % json.dumps(pf))
        if t2 is not None:
            secondary["mtp_T2"] = t2
            log("T=2: %s" % json.dumps(t2))

    if args.workload in ("all", "gguf") and pool:
        gg = bench_gguf(torch, Q, S, ctx, pool, X, out, idx)
        secondary["gguf_layer"] = gg
        log("gguf layer: %s" % json.dumps(gg))
    if cpu_cfg is not None and pool and mix == "q4k" and args.workload not in ("prefill", "mtp"):
        xh = X.cpu().numpy()
        cpu_cfg["q4k_matvec_512x2048"] = cpu_matvec(args.cpu_seconds * 0.05)
        cpu_cfg["decode_layer_q4k"] = cpu_decode_layer(pool[0], xh, args.cpu_seconds * 0.2,
                                                       "Q4_K / Q6_K")
        cpu_cfg["mtp_T2_q4k"] = cpu_two_tokens(pool[0], xh, args.cpu_seconds * 0.1)
    if cpu_cfg is not None and pool and args.workload == "iq2m":
        cpu_cfg["decode_layer_iq2m"] = cpu_decode_layer(pool[0], X.cpu().numpy(),
                                                        args.cpu_seconds * 0.2, "IQ2_M-mix")
    for L in pool:
        L.free()
    pool = []

    if args.workload == "all":
        log("building %d synthetic layers (iq2m)" % P)
        pool2 = [SynthLayer(ctx, 2000 + i, i, "iq2m") for i in range(P)]
        X2 = torch.empty(P, HIDDEN, dtype=torch.float32, device="cuda")
        for i in range(P):
            Q.synth_normal(X2[i], HIDDEN, 1.0, 78, S.stream_id(i, S.K_X))
        o2 = torch.empty_like(X2)
        i2 = torch.zeros(P, TOP_K, dtype=torch.int32, device="cuda")
        r2 = bench_decode(torch, Q, S, ctx, pool2, X2, o2, i2, args)
        if cpu_cfg is not None:
            cpu_cfg["decode_layer_iq2m"] = cpu_decode_layer(pool2[0], X2.cpu().numpy(),
                                                            args.cpu_seconds * 0.2, "IQ2_M-mix")
        r2["workload"] = ("decode layer, batch 1, IQ2_XXS gate/up, IQ3_S (even experts) / "
                          "IQ2_S (odd) down, F32 router, shared expert (Q4_K/Q6_K)")
        secondary["iq2m_decode"] = r2
        log("decode iq2m: %s" % json.dumps(r2))
        for L in pool2:
            L.free()
        # batched IQ layer: one IQ format per matrix kind, as in a GGUF expert pack
        pool3 = [SynthLayer(ctx, 2500 + i, i, "iq2a") for i in range(2)]
        pf3, _ = bench_prefill(torch, Q, S, ctx, pool3, args, with_t2=False,
                               formats=PREFILL_FORMATS["iq2a"])
        secondary["prefill_T%d_iq2xxs_iq3s" % args.prefill_tokens] = pf3
        log("prefill iq: %s" % json.dumps(pf3))
        for L in pool3:
            L.free()
        # batched layer of mixed per-expert formats (the decode IQ2_M mix):
        # one grouped launch per down format
        pool4 = [SynthLayer(ctx, 2600 + i, i, "iq2m") for i in range(2)]
        pf4, _ = bench_prefill(torch, Q, S, ctx, pool4, args, with_t2=False,
                               formats=PREFILL_FORMATS["iq2m"])
        secondary["prefill_T%d_iq2m_mixed" % args.prefill_tokens] = pf4
        log("prefill iq2m mixed: %s" % json.dumps(pf4))
        for L in pool4:
            L.free()
    if args.workload in ("all", "stack"):
        st = bench_stack(torch, Q, S, ctx, args, cpu=cpu_cfg)
        secondary["stack"] = st
        log("stack: %s" % json.dumps(st))
    if args.workload in ("all", "head"):
        hd = bench_head(torch, Q, S, ctx, args)
        secondary["output_head"] = hd
        log("output head: %s" % json.dumps(hd))
    if args.workload in ("all", "floor"):
        fl = bench_floor(torch, Q, ctx)
        secondary["kernel_floor"] = fl
        log("dependent-kernel floor: %s" % json.dumps(fl))

    if res_main is None:
        print(json.dumps({"secondary": secondary, "cpu_baselines": cpu_cfg}), flush=True)
        ctx.close()
        return

    # the headline's CPU figure: the same decode layer through the port
    cpu = None
    if cpu_cfg and mix in ("q4k", "iq2m"):
        head = cpu_cfg.get("decode_layer_%s" % mix)
        if head is not None:
            cpu = dict(head)
            cpu["host_cpu"] = host_cpu()

    kname = "k_moe_gate_up1"   # the gate/up kernel of one-token launches
    gk = res_main["kernels"][kname]
    achieved = gk["GBps"]
    traffic = None
    traffic_src = None
    if mix == "q4k" and os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as fh:
            tj = json.load(fh)
        if tj.get("kernel") == kname:
            traffic = tj.get("traffic_bytes_per_launch")
            traffic_src = os.path.relpath(TRAFFIC_FILE, HERE)
    res = {
        "metric": "decode MoE-FFN us/layer + HBM GB/s vs 8 TB/s peak; T=512 prefill TFLOP/s",
        "value": res_main["us_per_layer"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": res_main["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(res_main["us_per_layer"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "us_per_layer_spread": res_main["us_per_layer_spread"],
        "dtype": "f32",
        "data": "synthetic (seeded GGUF blocks generated on device)",
        "config": {"workload": "MoE FFN decode layer, batch 1: hidden 2048, 256 experts "
                               "top-8, inter 512, %s, F32 router, shared expert"
                               % ("Q4_K gate/up + Q6_K down" if mix == "q4k"
                                  else "IQ2_XXS gate/up + IQ3_S/IQ2_S down"),
                   "tokens_per_step": 1, "layer_pool": P},
        "hbm_GBps": res_main["hbm_GBps"],
        "hbm_frac": res_main["hbm_frac"],
        "bytes_per_step": res_main["bytes_per_step"],
        "eager_us_per_layer": res_main["eager_us_per_layer"],
        "kernels": res_main["kernels"],
        "dispatch_plan": res_main["dispatch_plan"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "kernel": kname,
                     "algorithmic_bytes": gk["bytes"], "avg_us": gk["us"],
                     "traffic_source": traffic_src},
        "cpu_baseline": cpu,
        "cpu_baselines": cpu_cfg,
        "secondary": secondary,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
