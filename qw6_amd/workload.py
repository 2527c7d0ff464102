"""Seeded synthetic MoE layers resident on the device.

Weights are generated in HBM by the library's synth kernels (the device twin
of qw6_amd.synth), expert matrices laid out as GGUF expert packs: expert e of
a pack at base + e * expert_bytes (bind_expert_pack, qw6.c:542-597), every
expert 256-byte aligned. Mixed per-expert quants (IQ3_S / IQ2_S downs) get
per-expert sizes in one pack.
"""
from __future__ import annotations

import numpy as np

from . import Context, make_layer
from . import synth as S
from . import synth_blocks, synth_normal

MIXES = {
    "q4k": (S.Q_Q4_K_M, lambda e: S.Q_Q6_K),
    "iq2m": (S.Q_IQ2_XXS, lambda e: S.Q_IQ3_S if e % 2 == 0 else S.Q_IQ2_S),
    # further K-quant combinations (format coverage of the batched path)
    "q5k": (S.Q_Q5_K, lambda e: S.Q_Q5_K),
    "q6q4": (S.Q_Q6_K, lambda e: S.Q_Q4_K_M),
    # one IQ format per matrix kind (as in a GGUF expert pack)
    "iq2a": (S.Q_IQ2_XXS, lambda e: S.Q_IQ3_S),
    "iq2b": (S.Q_IQ2_S, lambda e: S.Q_IQ2_S),
    # routed gate/up formats that differ by expert (qw6 keeps a tensor per
    # expert, qw6.h:160-162): IQ2_XXS / IQ3_S by parity with IQ3_S / IQ2_XXS
    # downs; Q5_K / Q4_K by parity (two occupancy classes of the grouped
    # kernels) with Q6_K downs
    "iqgu": (lambda e: S.Q_IQ2_XXS if e % 2 == 0 else S.Q_IQ3_S,
             lambda e: S.Q_IQ3_S if e % 2 == 0 else S.Q_IQ2_XXS),
    "q5q4": (lambda e: S.Q_Q5_K if e % 2 == 0 else S.Q_Q4_K_M, lambda e: S.Q_Q6_K),
}
SHARED_Q = (S.Q_Q4_K_M, S.Q_Q4_K_M, S.Q_Q6_K)
# shared expert formats where they differ from SHARED_Q: the same formats as
# the routed experts
SHARED_Q_MIX = {"q5k": (S.Q_Q5_K, S.Q_Q5_K, S.Q_Q5_K), "q6q4": (S.Q_Q6_K, S.Q_Q6_K, S.Q_Q4_K_M),
                "iq2b": (S.Q_IQ3_S, S.Q_IQ3_S, S.Q_IQ2_XXS)}


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


class SynthLayer:
    """One MoE layer generated on the device (torch uint8/float32 buffers)."""

    def __init__(self, ctx: Context, seed: int, layer: int = 0, mix: str = "q4k",
                 shared: bool = True, hidden: int = 2048, inter: int = 512,
                 n_experts: int = 256, top_k: int = 8, router: bool = True):
        import torch
        self.ctx, self.seed, self.layer, self.mix = ctx, seed, layer, mix
        self.hidden, self.inter, self.n_experts, self.top_k = hidden, inter, n_experts, top_k
        dev = torch.device("cuda", ctx.device)
        gq, down_fn = MIXES[mix]
        gate_fn = gq if callable(gq) else (lambda e: gq)
        self.quants = [(gate_fn(e), gate_fn(e), down_fn(e)) for e in range(n_experts)]
        shapes = ((inter, hidden), (inter, hidden), (hidden, inter))
        kinds = (S.K_GATE, S.K_UP, S.K_DOWN)
        self.packs, self.offsets, self.mats = [], [], []
        for k in range(3):
            sizes = [S.row_bytes(self.quants[e][k], shapes[k][1]) * shapes[k][0]
                     for e in range(n_experts)]
            offs = np.cumsum([0] + [_align(s) for s in sizes])
            buf = torch.empty(int(offs[-1]), dtype=torch.uint8, device=dev)
            for e in range(n_experts):
                q = self.quants[e][k]
                nb = shapes[k][0] * shapes[k][1] // 256
                synth_blocks(buf.data_ptr() + int(offs[e]), q, nb, seed,
                             S.stream_id(layer, kinds[k], e))
            self.packs.append(buf)
            self.offsets.append(offs)
            self.mats.append([(buf.data_ptr() + int(offs[e]), self.quants[e][k], shapes[k][0],
                               shapes[k][1]) for e in range(n_experts)])
        self.router = None
        if router:
            self.router = torch.empty(n_experts * hidden, dtype=torch.float32, device=dev)
            synth_normal(self.router, n_experts * hidden, 0.02, seed,
                         S.stream_id(layer, S.K_ROUTER))
        self.shared = None
        self.shared_bufs = []
        if shared:
            sh = []
            for k, q, kind in zip(range(3), SHARED_Q_MIX.get(mix, SHARED_Q),
                                  (S.K_SGATE, S.K_SUP, S.K_SDOWN)):
                r, c = shapes[k]
                buf = torch.empty(S.row_bytes(q, c) * r, dtype=torch.uint8, device=dev)
                synth_blocks(buf, q, r * c // 256, seed, S.stream_id(layer, kind))
                self.shared_bufs.append(buf)
                sh.append((buf.data_ptr(), q, r, c))
            self.shared = tuple(sh)
        self.experts = ctx.experts(*self.mats)
        self.desc = make_layer(hidden, inter, top_k, self.experts, router=self.router,
                               shared=self.shared)
        torch.cuda.synchronize()

    # ---- bytes a decode step must read -------------------------------------------
    def expert_bytes(self, e: int) -> int:
        shapes = ((self.inter, self.hidden), (self.inter, self.hidden), (self.hidden, self.inter))
        return sum(S.row_bytes(self.quants[e][k], shapes[k][1]) * shapes[k][0] for k in range(3))

    def shared_bytes(self) -> int:
        if self.shared is None:
            return 0
        return sum(S.row_bytes(m[1], m[3]) * m[2] for m in self.shared)

    # ---- host copies (for the oracle and the CPU baseline) --------------------------
    def expert_host(self, e: int):
        out = []
        shapes = ((self.inter, self.hidden), (self.inter, self.hidden), (self.hidden, self.inter))
        for k in range(3):
            q = self.quants[e][k]
            n = S.row_bytes(q, shapes[k][1]) * shapes[k][0]
            o = int(self.offsets[k][e])
            out.append((self.packs[k][o:o + n].cpu().numpy(), q))
        return tuple(out)

    def shared_host(self):
        if self.shared is None:
            return None
        return tuple((b.cpu().numpy(), m[1]) for b, m in zip(self.shared_bufs, self.shared))

    def router_host(self) -> np.ndarray:
        return self.router.cpu().numpy()

    def free(self):
        self.experts.free()
        self.packs = self.shared_bufs = []
        self.router = None


class SynthStack:
    """n_layers seeded MoE layers run as one decode step per token:
    h <- h + MoE_l(RMSNorm(h, w_l)) for l = 0 .. n_layers - 1 (qw6.c:2475-2484
    around qw6_apply_layer_moe, RMSNorm qw6.c:2503-2513), each layer one
    qw6_hip_moe_forward call with its norm weight fused in (norm_w) and the
    hidden state updated in place (x = residual = out).

    Layer l is SynthLayer(seed + l * seed_step, l, mix); its norm weight is
    N(1, 0.1) from (seed, stream (l, K_NORM)), generated on the device.
    """

    def __init__(self, ctx: Context, seed: int, n_layers: int, mix: str = "iq2m",
                 seed_step: int = 1, hidden: int = 2048, eps: float = 1e-6):
        import torch
        from . import MoeLayer
        self.ctx, self.seed, self.n_layers, self.hidden, self.eps = ctx, seed, n_layers, hidden, eps
        dev = torch.device("cuda", ctx.device)
        self.layers = [SynthLayer(ctx, seed + l * seed_step, l, mix, hidden=hidden)
                       for l in range(n_layers)]
        self.norm_w = torch.empty(n_layers, hidden, dtype=torch.float32, device=dev)
        self.descs = []
        for l, L in enumerate(self.layers):
            synth_normal(self.norm_w[l], hidden, 0.1, seed, S.stream_id(l, S.K_NORM), mean=1.0)
            d = MoeLayer.from_buffer_copy(L.desc)
            d.norm_w, d.norm_eps = self.norm_w[l].data_ptr(), eps
            self.descs.append(d)
        torch.cuda.synchronize()

    def step(self, h, idx, stream, hist=None):
        """One token through every layer, in place on h [1][hidden]; idx[l]
        receives layer l's selection. With hist, hist[l] receives h after
        layer l (a device copy on torch's current stream, which must be
        `stream`)."""
        for l in range(self.n_layers):
            self.ctx.moe_forward(self.descs[l], h, h, n_tok=1, residual=h, idx=idx[l],
                                 stream=stream)
            if hist is not None:
                hist[l].copy_(h[0])

    def capture(self, h, idx, hist=None):
        """The step captured as one HIP graph on a side stream (after one
        eager warm-up call); returns the graph."""
        import torch
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            self.step(h, idx, s.cuda_stream, hist)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                self.step(h, idx, s.cuda_stream, hist)
        torch.cuda.synchronize()
        return g

    def resident_bytes(self) -> int:
        return sum(sum(p.numel() for p in L.packs) for L in self.layers)

    def free(self):
        for L in self.layers:
            L.free()
        self.layers = []
