// qw6_hip.hip -- gfx950 kernels and C ABI of the routed-expert MoE FFN path.
//
// Decode path (fp32 accumulation), three kernels per MoE layer (a kernel
// boundary is the cheapest grid-wide dependency on this GPU):
//   k_moe_router : router GEMV over all experts (k_moe_router_w: two waves
//                  per expert row for one token), optional RMSNorm of the
//                  input, shared-expert gate weight.
//   k_moe_gate_up1: each workgroup takes one row tile of every selected
//                  expert and of the shared one, a wave per matrix pair (two
//                  for the shared pair on IQ layers at one token); each
//                  routed wave selects its own expert from the logits (softmax
//                  top-k), then streams its gate/up rows into LDS with
//                  direct-to-LDS 16-byte loads, dequantizing step s while step
//                  s+1 is in flight; writes silu(gate) * up. Wave 0 of
//                  workgroup 0 routes fully and publishes the slot table.
//   k_moe_down   : one workgroup per tile of output rows, one wave per
//                  selected expert (plus the shared one); per-expert row sums
//                  meet in LDS and are combined in selection order, with the
//                  residual -- no atomics, deterministic.
// A launch of several tokens (up to 16) runs the same kernels with one row of
// the grid per token (token_view): each token's workgroups do exactly a
// one-token call's work, and a token's workgroup b shares an XCD with every
// other token's workgroup b, so experts that several tokens select, and the
// shared expert, are read from HBM about once. In the automatic mode, calls
// of 17 tokens or more (16 for layers holding IQ formats) take the grouped
// bf16-MFMA kernels of qw6_prefill.hip (one launch per expert format
// present); mode 3 runs the small-batch MFMA kernels k_mx_* in launches of up
// to 4 tokens.
// Routing never leaves the device (qw6's Vulkan path reads idx/w back to the
// host per layer, qw6_vk.c:3371-3374).
//
// Lane mapping: a row of K columns has U = K/32 units of 32 weights
// (qw6_dev.h); a wave covers 64/U rows per step with lane -> (row, unit)
// fixed, so each lane keeps its unit's activations in registers across rows,
// and the rows of one step are always 8 GGUF blocks (<= 1680 bytes).

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "../../include/qw6_hip.h"
#include "qw6_dev.h"
#include "qw6_host.h"
#include "qw6_moe.h"
#include "qw6_tile.h"

using namespace qw6;

namespace {

__device__ const IqTables g_tabs = make_tables();

constexpr int kWG = 256;           // threads per workgroup (4 waves)
constexpr uint32_t kMaxTok = 4;         // tokens per launch of the small-batch MFMA kernels
constexpr uint32_t kSplitMaxTok = 16;   // tokens per launch of the fp32 kernels (one grid row each)
// waves per router row for one token (hidden 512 to 2048): two halve each
// wave's loads and sums (the 40-layer stack with its fused norm 17.70 ->
// 17.35 us per layer; four measured the same as two)
constexpr int kRouterWaves = 2;
// Automatic switch to the grouped MFMA path: calls of this many tokens or
// more (where the two paths' timings cross on one MI355X: Q4_K / Q6_K
// layers past the 16 tokens of one launch, layers holding IQ formats at 16)
constexpr uint32_t kGroupedMinTokens = 17;
constexpr uint32_t kGroupedMinTokensIq = 16;
constexpr uint32_t kLdsBudget = 64 * 1024;   // dynamic LDS per workgroup
constexpr uint32_t kMxLdsBudget = 150 * 1024;   // k_mx_*: gfx950 has 160 KB per workgroup
constexpr int kProfEv = 6;         // events per profiled MoE call (3 kernels x start/stop)

thread_local char g_err[512];
#ifdef QW6_TRACE
// Per-workgroup wall-clock spans of the MoE kernels (instrumented builds
// only): g_trace[kernel][block] = {start, end} of wave 0, 100 MHz ticks.
__device__ unsigned long long g_trace[4][4096][2];
struct TraceScope {
    int k;
    __device__ explicit TraceScope(int k_) : k(k_) {
        if (threadIdx.x == 0 && blockIdx.x < 4096) g_trace[k][blockIdx.x][0] = wall_clock64();
    }
    __device__ ~TraceScope() {
        if (threadIdx.x == 0 && blockIdx.x < 4096) g_trace[k][blockIdx.x][1] = wall_clock64();
    }
};
#define TRACE_SCOPE(k) TraceScope trace_scope_(k)
__device__ unsigned long long g_mark[4][4096][6];
#ifdef QW6_TRACE_MARKS
#ifndef QW6_MARK_TID
#define QW6_MARK_TID 0
#endif
// Phase marks: the clock of thread QW6_MARK_TID when it reaches the mark (no
// added wait: a mark placed after a use of loaded data records when that data
// arrived). Diagnostic builds only.
#define TRACE_MARK(k, i)                                                            \
    do {                                                                            \
        if (threadIdx.x == QW6_MARK_TID && blockIdx.x < 4096)                       \
            g_mark[k][blockIdx.x][i] = wall_clock64();                              \
    } while (0)
#else
#define TRACE_MARK(k, i) do {} while (0)
#endif
#define TRACE_MARK_IF(c, k, i) \
    do {                       \
        if (c) TRACE_MARK(k, i); \
    } while (0)
#else
#define TRACE_SCOPE(k)
#define TRACE_MARK(k, i)
#define TRACE_MARK_IF(c, k, i)
#endif


int vfail(const char* fmt, va_list ap) {
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    fprintf(stderr, "qw6_hip: %s\n", g_err);
    return -1;
}

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const int r = vfail(fmt, ap);
    va_end(ap);
    return r;
}

#define CK(expr)                                                                   \
    do {                                                                           \
        hipError_t _e = (expr);                                                    \
        if (_e != hipSuccess)                                                      \
            return fail("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),    \
                        __FILE__, __LINE__);                                       \
    } while (0)


// ---- staging: global bytes -> LDS ----------------------------------------------

// Copy `bytes` (even) from 16-byte-aligned global src to 16-byte-aligned LDS
// dst with the waves [w0, w0 + nw) of the workgroup: 16-byte direct-to-LDS
// loads (gfx950 global_load_lds_dwordx4; a wave's 64 lanes fill 1 KB) for the
// body, 2-byte copies for the tail. Waves outside the range return at once.
// The caller waits (stage_wait / wave_wait) before reading.
__device__ __forceinline__ void stage(uint8_t* dst, const uint8_t* src, uint32_t bytes,
                                      uint32_t w0 = 0, uint32_t nw = 0xffffu) {
    const uint32_t wave = (threadIdx.x >> 6) - w0, lane = threadIdx.x & 63u;
    const uint32_t nwv = min(nw, (uint32_t)(blockDim.x >> 6));
    if (wave >= nwv) return;
    const uint32_t n16 = bytes >> 4;
    for (uint32_t c0 = wave * 64; c0 < n16; c0 += nwv * 64) {
        const uint32_t c = c0 + lane;
        if (c < n16)
            __builtin_amdgcn_global_load_lds((glb_void_t*)(src + 16ull * c),
                                             (lds_void_t*)(dst + 16u * c0), 16, 0, 0);
    }
    const uint32_t rem = (bytes & 15u) >> 1;
    if (wave == 0 && lane < rem) {
        const uint16_t v = ((const uint16_t*)(src + 16ull * n16))[lane];
        ((uint16_t*)(dst + 16u * n16))[lane] = v;
    }
}

__device__ __forceinline__ void wave_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier without a memory fence, for LDS data whose writers have
// each waited for their own LDS-direct loads (vmcnt) before it: the global
// loads a wave still has in flight stay in flight (__syncthreads would wait
// for all of them). The memory clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void stage_wait() {
    wave_wait();
    __syncthreads();
}

// Lattice tables needed by `mask` into LDS (IqTables layout at tab), by the
// waves [w0, 4) of a 4-wave block (all waves of any block when w0 == 0).
__device__ __forceinline__ void stage_tables_from(uint8_t* tab, uint32_t mask, uint32_t w0) {
    const uint8_t* g = (const uint8_t*)&g_tabs;
    const uint32_t nw = w0 ? 4u - w0 : 0xffffu;
    if (mask & 1u) stage(tab, g, kTabOffSgn8, w0, nw);   // IQ2_XXS signs + grid
    if (mask & 6u) stage(tab + kTabOffSgn8, g + kTabOffSgn8, kTabOffIq3s - kTabOffSgn8, w0, nw);
    if (mask & 4u) stage(tab + kTabOffIq3s, g + kTabOffIq3s, kTabOffIq2s - kTabOffIq3s, w0, nw);
    if (mask & 2u) stage(tab + kTabOffIq2s, g + kTabOffIq2s, kTabBytes - kTabOffIq2s, w0, nw);
}
__device__ __forceinline__ void stage_tables(uint8_t* tab, uint32_t mask) {
    stage_tables_from(tab, mask, 0);
}

__host__ __device__ inline uint32_t tab_bytes(uint32_t mask) {
    return mask & 2u ? kTabBytes : mask & 4u ? kTabOffIq2s : mask & 1u ? kTabOffSgn8 : 0u;
}

__host__ __device__ inline uint32_t align16(uint32_t n) { return (n + 15u) & ~15u; }

// ---- one matrix tile: per-row dot products --------------------------------------


// Row tile staged in LDS at byte offset tile_off (rows [0, rows_valid)).
// Wave `wave` owns S steps of rps = 64/U rows: local row of step s for lane
// group q = lane/U is (wave*S + s)*rps + q. Each lane accumulates its unit's
// partial sums for all S steps, then one reduce-scatter per token leaves step
// scatter_step<S>(lane) on each lane; emit(row, value[T]) runs on the first
// lane of each sub-group that owns a row.
template <int T, int S, int FF, typename Emit>
__device__ __forceinline__ void tile_rows(int f_rt, const uint32_t* lds, uint32_t tile_off,
                                          uint32_t rb, uint32_t K, const float (&xr)[T][32],
                                          const float (&sx)[T][4], uint32_t rows_valid,
                                          uint32_t wave, Emit emit) {
    const int f = FF >= 0 ? FF : f_rt;
    const uint32_t U = K >> 5, rps = 64 / U;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t unit = lane & (U - 1), blk = unit >> 3, q = lane / U;
    const int j = (int)(unit & 7);
    const uint32_t bb = fmt_block_bytes(f);
    float acc[T][S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t rl = (wave * S + s) * rps + q;
        float a[T];
#pragma unroll
        for (int t = 0; t < T; t++) a[t] = 0.f;
        if (rl < rows_valid) unit_dot<T>(f, lds, tile_off + rl * rb + blk * bb, j, lds, xr, sx, a);
#pragma unroll
        for (int t = 0; t < T; t++) acc[t][s] = a[t];
    }
    float r[T];
#pragma unroll
    for (int t = 0; t < T; t++) r[t] = reduce_scatter_c<S>(acc[t], U);
    const uint32_t s = scatter_step<S>(lane, U);
    const uint32_t rl = (wave * S + s) * rps + q;
    if ((unit & (U / S - 1)) == 0 && rl < rows_valid) emit(rl, r);
}

template <int T, int FF>
__device__ __forceinline__ void load_x_all(int f_rt, const float* x, uint32_t ldx, uint32_t K,
                                           float (&xr)[T][32]) {
    const int f = FF >= 0 ? FF : f_rt;
    const uint32_t U = K >> 5;
    const uint32_t unit = (threadIdx.x & 63) & (U - 1);
#pragma unroll
    for (int t = 0; t < T; t++) load_unit_x(f, x + (size_t)t * ldx, unit >> 3, (int)(unit & 7), xr[t]);
}

template <int T>
__device__ __forceinline__ void x_sums_all(int f, const float (&xr)[T][32], float (&sx)[T][4]) {
#pragma unroll
    for (int t = 0; t < T; t++) unit_x_sums(f, xr[t], sx[t]);
}

// ---- single-matrix matvec --------------------------------------------------------

constexpr int kStepsMv = 4;

template <int T, int FF>
__global__ __launch_bounds__(kWG) void k_matvec(MatD W, const float* __restrict__ x,
                                                float* __restrict__ y, uint32_t R,
                                                uint32_t tmask) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t r0 = blockIdx.x * R;
    const uint32_t nv = min(R, W.rows - r0);
    const uint32_t toff = tab_bytes(tmask);
    const uint32_t xoff = toff + align16(R * W.rb) + 16;
    stage_tables(smem, tmask);
    stage(smem + toff, W.p + (size_t)r0 * W.rb, nv * W.rb);
    stage(smem + xoff, (const uint8_t*)x, T * W.cols * 4);
    stage_wait();
    const uint32_t* s = (const uint32_t*)smem;
    float xr[T][32], sx[T][4];
    load_x_all<T, FF>(W.fmt, (const float*)(smem + xoff), W.cols, W.cols, xr);
    x_sums_all<T>(FF >= 0 ? FF : W.fmt, xr, sx);
    tile_rows<T, kStepsMv, FF>(W.fmt, s, toff, W.rb, W.cols, xr, sx, nv, threadIdx.x >> 6,
                           [&](uint32_t rl, const float(&v)[T]) {
#pragma unroll
                               for (int t = 0; t < T; t++) y[(size_t)t * W.rows + r0 + rl] = v[t];
                           });
}

// Any K multiple of 256: one wave per row, lanes stride over the units, the
// row staged in LDS, activations read from global memory per unit.
template <int T>
__global__ __launch_bounds__(64) void k_matvec_generic(MatD W, const float* __restrict__ x,
                                                       float* __restrict__ y, uint32_t tmask) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t r = blockIdx.x;
    const uint32_t toff = tab_bytes(tmask);
    const uint32_t lane = threadIdx.x;
    stage_tables(smem, tmask);
    stage(smem + toff, W.p + (size_t)r * W.rb, W.rb);
    stage_wait();
    const uint32_t* s = (const uint32_t*)smem;
    const uint32_t U = W.cols >> 5, bb = fmt_block_bytes(W.fmt);
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.f;
    for (uint32_t u = lane; u < U; u += 64) {
        const uint32_t blk = u >> 3;
        const int j = (int)(u & 7);
        float xr[T][32], sx[T][4];
#pragma unroll
        for (int t = 0; t < T; t++) {
            load_unit_x(W.fmt, x + (size_t)t * W.cols, blk, j, xr[t]);
            unit_x_sums(W.fmt, xr[t], sx[t]);
        }
        unit_dot<T>(W.fmt, s, toff + blk * bb, j, s, xr, sx, acc);
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float v = group_sum<64>(acc[t]);
        if (lane == 0) y[(size_t)t * W.rows + r] = v;
    }
}

// F32 rows: one wave per row.
template <int T>
__global__ __launch_bounds__(64) void k_matvec_f32(const float* __restrict__ w,
                                                   const float* __restrict__ x,
                                                   float* __restrict__ y, uint32_t rows,
                                                   uint32_t cols) {
    const uint32_t r = blockIdx.x, lane = threadIdx.x;
    const float* wr = w + (size_t)r * cols;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.f;
    for (uint32_t c = lane; c < cols; c += 64) {
        const float wv = wr[c];
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = fmaf(wv, x[(size_t)t * cols + c], acc[t]);
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float v = group_sum<64>(acc[t]);
        if (lane == 0) y[(size_t)t * rows + r] = v;
    }
}

// ---- routing (wave_route: qw6_dev.h) -----------------------------------------------

__global__ __launch_bounds__(64) void k_route(const float* __restrict__ logits, uint32_t n,
                                              uint32_t top_k, uint32_t* idx, float* w) {
    __shared__ uint2 scr[kRouteScr];
    const uint32_t t = blockIdx.x;
    wave_route(logits + (size_t)t * n, n, top_k, scr, idx + t * top_k, w + t * top_k);
}

// ---- MoE decode kernels --------------------------------------------------------------
//
// Three kernels per layer (a kernel boundary is the cheapest grid-wide
// dependency on this GPU; in-kernel grid barriers cost several times more):
//   k_moe_router : router GEMV, one wave per expert row, or two in
//                  k_moe_router_w (+ optional RMSNorm of the input, + the
//                  shared-expert gate weight).
//   k_moe_gate_up1: every selected expert's gate/up rows of one row tile per
//                  workgroup, each routed wave routing the token itself from
//                  the logits (1 KB per token); silu(gate) * up -> mid.
//                  Workgroup 0 also publishes the slot table (selected
//                  experts resolved to matrices).
//   k_moe_down   : one workgroup per tile of output rows, one wave per
//                  selected expert (the shared one first, it needs no routing);
//                  row sums meet in LDS and are combined in a fixed order with
//                  the residual -- no atomics, deterministic.

constexpr int kStepsGu = 2;     // row steps per wave, gate/up
constexpr int kStepsDn = 2;     // row steps per wave, down
constexpr uint32_t kMaxSlots = kMaxTok * 8;
constexpr uint32_t kSlotBytes = 2048;   // LDS slot of one step group (8 blocks <= 1680 B)
// rows of inter floats in the mid workspace: the small-batch kernels' (max_u + 1)
// x T, the fp32 kernels' (top_k + 1) per token
constexpr uint32_t kMidRows = (kMaxSlots + 1) * kMaxTok > 9 * kSplitMaxTok ? (kMaxSlots + 1) * kMaxTok
                                                                           : 9 * kSplitMaxTok;

// The slot table the gate/up kernels publish for the down kernels: distinct
// selected experts in first-use order with their down matrix and per-token
// weights (k_moe_gate_up1: one table per token, the selection itself).
struct SlotTable {
    uint32_t n;                    // number of slots in use
    uint32_t pad[3];
    const uint8_t* p[kMaxSlots];   // down matrix of slot u
    int32_t fmt[kMaxSlots];
    uint32_t rb[kMaxSlots];
    float wt[kMaxSlots][kMaxTok];  // gate weight of slot u for token t (0: unused)
};

struct MoeArgs {
    uint32_t hidden, inter, n_experts, top_k, T, max_u;
    const float* x;               // layer input [T][hidden]
    const float* xin;             // input of the expert matvecs (x or its RMSNorm)
    const float* router;          // F32 router or nullptr
    const float* route_logits;    // logits the routing reads (workspace or given)
    const float* shared_router;   // nullptr: shared weight 1
    const float* norm_w;          // RMSNorm weight or nullptr
    float norm_eps;
    uint32_t n_sh_wg;             // shared-expert workgroups in k_mx_gate_up
    const ExpertEnt* experts;
    PackRef pk[3];
    MatD sg, su, sd;              // shared expert; sg.p == nullptr: none
    float* logits;                // [T][n_experts] workspace
    float* xn;                    // [T][hidden] normalised input (norm_w set)
    float* sw;                    // [T] shared weight (written when shared_router)
    SlotTable* slots;
    float* mid;                   // [(max_u + 1)][T][inter], shared expert at max_u
    const float* residual;
    float* out;
    uint32_t* idx_out;
    float* w_out;
    uint32_t tmask_gu, tmask_dn;
    uint32_t gu_pb;               // k_moe_gate_up1: LDS bytes of one (gate, up) step pair
    int xl_dn;                    // a format with every routed down matrix's
                                  // activation layout, or -1 (x_layout)
    // small-batch MFMA path (k_mx_*): operands of the expert input and of mid
    uint4* xa;                    // [hidden / 32][64]; k_moe_router writes it when set
    uint16_t* xs;                 // [hidden / 256][2][4][3][8]
    uint4* ma;                    // [max_u + 1][inter / 32][64], shared expert last
    uint16_t* ms;                 // [max_u + 1][inter / 256][2][4][3][8]
    uint32_t mx_gu_soff;          // k_mx_gate_up: LDS offset of the staged blocks
    uint32_t mx_sb;               // k_mx_down: LDS bytes of one staged block
    uint32_t mx_nsl;              // k_mx_down: staged blocks per round
};

// k_moe_gate_up1 and k_moe_down<1> launched for several tokens hold token t's
// workgroups at blockIdx.y = t (one token per row of the grid, so a token's
// workgroup b still runs on XCD b % 8). a becomes token t's view: the
// buffers the kernels always have offset as for a one-token call of its own
// (slot table t, its (max_u + 1) x inter block of mid, max_u = top_k); the
// optional ones (residual, idx_out, w_out) are offset where they are used,
// so no branch on them delays the first loads. One-token launches have t = 0.
__device__ __forceinline__ void token_view(MoeArgs& a) {
    const uint32_t t = blockIdx.y;
    a.route_logits += (size_t)t * a.n_experts;
    a.xin += (size_t)t * a.hidden;
    a.out += (size_t)t * a.hidden;
    a.sw += t;
    a.slots += t;
    a.mid += (size_t)t * (a.max_u + 1) * a.inter;
}

// Addresses are formed from an index below n_experts whatever the routing
// gave (a routing result is always below it; the bound keeps every weight
// read inside the layer's experts by construction).
__device__ __forceinline__ MatD expert_mat(const MoeArgs& a, uint32_t e, int k) {
    const PackRef& P = a.pk[k];
    const uint32_t rows = k < 2 ? a.inter : a.hidden, cols = k < 2 ? a.hidden : a.inter;
    e = min(e, a.n_experts - 1u);
    if (P.regular) return MatD{P.base + P.stride * e, P.fmt, rows, cols, P.rb};
    const ExpertEnt& E = a.experts[e];
    return MatD{E.p[k], E.fmt[k], rows, cols, E.rb[k]};
}
// The same for an expert index e that is equal on every lane of the wave.
// The table does not change during a launch: read through the constant
// address space, the uniform index gives scalar loads, which a later wait on
// vector loads does not have to cover.
__device__ __forceinline__ MatD expert_mat_wave(const MoeArgs& a, uint32_t e, int k) {
    const PackRef& P = a.pk[k];
    const uint32_t rows = k < 2 ? a.inter : a.hidden, cols = k < 2 ? a.hidden : a.inter;
    e = min((uint32_t)__builtin_amdgcn_readfirstlane(e), a.n_experts - 1u);
    if (P.regular) return MatD{P.base + P.stride * e, P.fmt, rows, cols, P.rb};
    using CE = __attribute__((address_space(4))) const ExpertEnt;
    const CE& E = ((CE*)a.experts)[e];
    return MatD{E.p[k], E.fmt[k], rows, cols, E.rb[k]};
}

// Format template argument of the expert kernels: F >= 0 one format known
// at compile time; -1 any of the six (a switch per matrix); F <= -2 the set
// of formats in the mask -(F + 2) (bit f: format f), a switch over those
// only. A layer mixes two or three formats, and a switch over all six makes
// the kernel three to six times the code of a one-format one.
__host__ __device__ constexpr bool fmt_in(int FS, int f) {
    return FS >= 0 ? FS == f : FS == -1 ? true : (((uint32_t)(-(FS + 2)) >> f) & 1u) != 0;
}
__host__ __device__ constexpr int fmt_set(uint32_t mask) { return -(int)mask - 2; }

// fn(std::integral_constant<int, f>) for the runtime format f, compiled for
// the formats of the set FS only (another f does nothing: the host passes the
// set of the formats the layer holds).
template <int FS, typename Fn>
__device__ __forceinline__ void by_fmt(int f, Fn fn) {
    switch (f) {
    case F_Q4K: if constexpr (fmt_in(FS, F_Q4K)) fn(std::integral_constant<int, F_Q4K>{}); break;
    case F_Q5K: if constexpr (fmt_in(FS, F_Q5K)) fn(std::integral_constant<int, F_Q5K>{}); break;
    case F_Q6K: if constexpr (fmt_in(FS, F_Q6K)) fn(std::integral_constant<int, F_Q6K>{}); break;
    case F_IQ2XXS: if constexpr (fmt_in(FS, F_IQ2XXS)) fn(std::integral_constant<int, F_IQ2XXS>{}); break;
    case F_IQ2S: if constexpr (fmt_in(FS, F_IQ2S)) fn(std::integral_constant<int, F_IQ2S>{}); break;
    default: if constexpr (fmt_in(FS, F_IQ3S)) fn(std::integral_constant<int, F_IQ3S>{}); break;
    }
}

// Stage one step group (the rows one wave step covers: 8 GGUF blocks, a
// multiple of 16 bytes, <= 1680 B) into a 2 KB LDS slot with exactly two
// 16-byte direct-to-LDS loads per lane. Lanes past the group's end reload the
// group's first chunk into the unused tail of the slot, so every wave issues
// the same number of loads and the step waits below can use immediates.
__device__ __forceinline__ void stage_group(uint8_t* slot, const uint8_t* src, uint32_t bytes) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n16 = bytes >> 4;
#pragma unroll
    for (uint32_t i = 0; i < 2; i++) {
        const uint32_t c = 64u * i + lane;
        const uint32_t cc = c < n16 ? c : 0u;
        __builtin_amdgcn_global_load_lds((glb_void_t*)(src + 16ull * cc),
                                         (lds_void_t*)(slot + 1024u * i), 16, 0, 0);
    }
}

// Loads per lane that stage one (gate, up) step pair of format f (2 x 8 blocks).
__host__ __device__ constexpr uint32_t pair_loads(int f) { return (16u * fmt_block_bytes(f) + 1023u) / 1024u; }

// Stage the step groups g (gate) and u (up) of gbytes each (8 blocks, a
// multiple of 16 bytes) into one LDS pair slot, gate at +0 and up at +gbytes,
// with nl 16-byte direct-to-LDS loads per lane (the slot holds exactly the
// pair's 2 gbytes).
__device__ __forceinline__ void stage_pair(uint8_t* slot, const uint8_t* g, const uint8_t* u,
                                           uint32_t gbytes, uint32_t nl) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n16 = gbytes >> 4;
    for (uint32_t i = 0; i < nl; i++) {
        const uint32_t c = 64u * i + lane;
        const uint8_t* src = c < n16 ? g + 16ull * c : u + 16ull * (c - n16);
        // lanes past the pair's end stay idle (every load has an active
        // lane: nl = ceil(2 n16 / 64)), so the slot is the pair's bytes
        if (c < 2 * n16)
            __builtin_amdgcn_global_load_lds((glb_void_t*)src, (lds_void_t*)(slot + 1024u * i), 16, 0, 0);
    }
}

// Wait until at most n of this wave's vector-memory loads are outstanding
// (n a compile-time constant after unrolling). An s_waitcnt instruction the
// compiler knows of: it counts the wait in its own bookkeeping, so later uses
// of those loads' registers get no stricter wait of its making. gfx9
// encoding: vmcnt bits 3:0 and 15:14; expcnt (7) and lgkmcnt (15) not waited.
#define QW6_VMCNT(n) (((n) & 15u) | (((n) >> 4) << 14) | 0xf70u)
__device__ __forceinline__ void wait_vm(uint32_t n) {
    switch (n) {
    case 2: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(2u)); break;
    case 3: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(3u)); break;
    case 4: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(4u)); break;
    case 6: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(6u)); break;
    case 8: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(8u)); break;
    case 9: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(9u)); break;
    case 10: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(10u)); break;
    case 12: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(12u)); break;
    case 14: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(14u)); break;
    case 16: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(16u)); break;
    case 20: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(20u)); break;
    case 24: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(24u)); break;
    case 28: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(28u)); break;
    case 32: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(32u)); break;
    case 36: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(36u)); break;
    default: __builtin_amdgcn_s_waitcnt(QW6_VMCNT(0u)); break;
    }
    // compiler barrier: no memory access (the LDS reads of what the waited
    // loads wrote, in particular) moves across the wait
    asm volatile("" ::: "memory");
}

// Routing of all T tokens inside one workgroup: wave t routes token t; the
// distinct selected experts are numbered in first-use order ("slots").
// Leaves s_slot_e[u] (expert of slot u), s_wt[u][t] (gate weight of slot u
// for token t, 0 if unused), s_idx / s_w (per-token selection) and *s_n.
// keys: token `wave`'s logit keys, loaded by route_keys in waves < T.
template <int T>
__device__ __forceinline__ void route_prologue(const MoeArgs& a, uint32_t (&keys)[4], uint2* scr,
                                               uint32_t* s_idx, float* s_w,
                                               uint32_t* s_slot_e, float* s_wt, uint32_t* s_n) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (T == 1) {   // one token: the slots are the selection itself
        if (wave == 0) {
            wave_route_keys(keys, a.top_k, scr, s_idx, s_w);
            __builtin_amdgcn_wave_barrier();
            if (lane < a.top_k) {
                s_slot_e[lane] = s_idx[lane];
                s_wt[lane * kMaxTok] = s_w[lane];
#pragma unroll
                for (uint32_t t = 1; t < kMaxTok; t++) s_wt[lane * kMaxTok + t] = 0.f;
            }
            if (lane == 0) *s_n = a.top_k;
        }
        __syncthreads();
        return;
    }
    if (wave < (uint32_t)T)
        wave_route_keys(keys, a.top_k, scr + wave * kRouteScr, s_idx + wave * a.top_k, s_w + wave * a.top_k);
    __syncthreads();
    if (wave == 0) {
        const uint32_t ne = T * a.top_k;
        const uint32_t e = lane < ne ? s_idx[lane] : 0xffffffffu;
        uint32_t first = lane;
        if (T > 1)
            for (uint32_t j = 0; j < lane && lane < ne; j++)
                if (s_idx[j] == e) { first = j; break; }
        const bool is_first = lane < ne && first == lane;
        const uint64_t mask = __ballot(is_first);
        const uint32_t slot = __popcll(mask & ((1ull << first) - 1ull));
        for (uint32_t i = lane; i < kMaxSlots * kMaxTok; i += 64) s_wt[i] = 0.f;
        if (is_first) s_slot_e[slot] = e;
        if (lane == 0) *s_n = (uint32_t)__popcll(mask);
        __builtin_amdgcn_wave_barrier();
        // A token selects one expert at several ranks only once its logits
        // are down to -inf and NaN (index 0 again, qw6.c:2808-2816); those
        // later ranks weigh exactly 0 (or NaN, with every weight NaN), so the
        // first rank of the expert in the token writes the sum over its ranks
        // and qw6's sum w_k * y_k is kept. One writer per (slot, token).
        if (lane < ne) {
            const uint32_t k0 = lane - lane % a.top_k;
            bool first_in_tok = true;
            float wsum = 0.f;
            for (uint32_t j = k0; j < k0 + a.top_k; j++) {
                if (s_idx[j] != e) continue;
                if (j < lane) first_in_tok = false;
                wsum += s_w[j];
            }
            if (first_in_tok) s_wt[slot * kMaxTok + lane / a.top_k] = wsum;
        }
    }
    __syncthreads();
}

// ---- small-batch MFMA operands -------------------------------------------------------
// The k_mx_* kernels multiply GGUF blocks decoded into bf16 MFMA operands
// (qw6_tile.h) with the tokens as the 16 rows of the A operand: row m = 4 t + p
// holds part p of token t's activation, p = 0, 1, 2 the bf16 hi / mid / lo
// parts (their sum is the fp32 value to within 2^-24 of it); rows p = 3 and
// t >= T are zero, so D[m][n] summed over p is token t's product with row n.
//  - Sub-block operands (xa, ma): one 1 KB entry per 32-column sub-block;
//    lane l = 16 q + m holds columns 8 q .. 8 q + 7 of row m.
//  - Half-sum operands (xs, ms): per 256-column block, half (columns 0-15 or
//    16-31 of each of its 8 sub-blocks) and token, the 3 bf16 parts of the 8
//    half-sums, [block][half][t][part][sub-block]: the bias and minimum
//    corrections take them in k-slots 8 part + sub-block (mx_load_a).

// Part p (0: hi, 1: mid, 2: lo, 3: none) of v as bf16 bits.
__device__ __forceinline__ uint32_t bf16_part(float v, uint32_t p) {
    const __bf16 h = (__bf16)v;
    const float r1 = v - (float)h;
    const __bf16 m = (__bf16)r1;
    const __bf16 l = (__bf16)(r1 - (float)m);
    return p == 0 ? bfb(h) : p == 1 ? bfb(m) : p == 2 ? bfb(l) : 0u;
}

// Sub-block operand lane of eight values (columns 8 q .. 8 q + 7 of row m = 4 t + p).
__device__ __forceinline__ uint4 mx_pack8(const float (&v)[8], uint32_t p) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = bf16_part(v[2 * i], p) | (bf16_part(v[2 * i + 1], p) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// The 3 bf16 parts of half-sum hs of sub-block sb, half h, token t, into a
// half-sum operand array of nkb blocks.
__device__ __forceinline__ void mx_put_halfsum(uint16_t* dst, uint32_t sb, uint32_t h, uint32_t t, float hs) {
    uint16_t p3[3];
    split3(hs, p3);
    uint16_t* o = dst + (((size_t)(sb >> 3) * 2 + h) * 4 + t) * 24 + (sb & 7u);
    o[0] = p3[0];
    o[8] = p3[1];
    o[16] = p3[2];
}

// Operands of input sub-block e (one wave): the activations as the expert
// kernels see them (RMSNorm applied with scale sc, this lane's token's, as the
// per-token kernels' input), split into parts, and the two half-sums per token.
template <int T>
__device__ __forceinline__ void mx_input_operands(const MoeArgs& a, uint32_t e, float sc) {
    const uint32_t lane = threadIdx.x & 63u, m = lane & 15u, q = lane >> 4, t = m >> 2, p = m & 3u;
    const uint32_t c0 = 32u * e + 8u * q;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.f;
    if (t < (uint32_t)T) {
        const float4* xr = (const float4*)(a.x + (size_t)t * a.hidden + c0);
        const float4 x0 = xr[0], x1 = xr[1];
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
        if (a.norm_w) {
            const float4* wr = (const float4*)(a.norm_w + c0);
            const float4 w0 = wr[0], w1 = wr[1];
            const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = v[i] * sc * w[i];
        }
    }
    a.xa[(size_t)e * 64 + lane] = mx_pack8(v, p);
    float hs = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) hs += v[i];
    hs += __shfl_xor(hs, 16);   // lanes q and q ^ 1: the half q / 2
    if (p == 0 && (q & 1u) == 0) mx_put_halfsum(a.xs, e, q >> 1, t, hs);
}

// The expert of slot u (the u-th distinct selected expert in first-use order
// over tokens, then ranks, as route_prologue numbers them) for a block that
// publishes nothing: waves t < T rank token t's logits (route_rank; no gate
// weights), then every wave finds the slot from the T * top_k selections
// with lane reads -- one barrier. Returns false if fewer than u + 1 slots.
// scr: T * kRouteScr routing scratch, s_sel: T * top_k words (LDS).
template <int T>
__device__ __forceinline__ bool route_slot_select(const MoeArgs& a, uint32_t (&keys)[4], uint32_t u,
                                                  uint32_t& e_out, uint2* scr, uint32_t* s_sel) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (wave < (uint32_t)T) {
        uint2 me2;
        uint32_t rank, ncand;
        if (route_rank(keys, a.top_k, scr + wave * kRouteScr, me2, rank, ncand)) {
            if (lane < ncand && rank < a.top_k)   // only -inf left: qw6 picks index 0
                s_sel[wave * a.top_k + rank] = me2.y > kKeyNegInf ? ~me2.x : 0u;
            // ranks without a candidate (NaN logits are never candidates) are
            // taken once only -inf and NaN are left: index 0, as in
            // wave_route_keys. Candidates hold ranks [0, ncand), so these
            // lanes write the other ranks and no slot is written twice.
            if (lane >= ncand && lane < a.top_k) s_sel[wave * a.top_k + lane] = 0u;
        } else if (lane < a.top_k) {
            const uint2 me = scr[wave * kRouteScr + 32 + lane];
            s_sel[wave * a.top_k + lane] = me.y > kKeyNegInf ? ~me.x : 0u;
        }
    }
    __syncthreads();
    const uint32_t ne = T * a.top_k;
    const uint32_t e = lane < ne ? s_sel[lane] : 0xffffffffu;
    uint32_t first = lane;
    for (uint32_t j = 0; j < ne; j++) {
        const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)e, (int)j);
        if (j < first && v == e) first = j;
    }
    const bool is_first = lane < ne && first == lane;
    const uint64_t mask = __ballot(is_first);
    const uint32_t slot = __popcll(mask & ((1ull << lane) - 1ull));
    const uint64_t hit = __ballot(is_first && slot == u);
    if (!hit) return false;
    e_out = (uint32_t)__builtin_amdgcn_readlane((int)e, __ffsll((unsigned long long)hit) - 1);
    return true;
}

// x (T tokens) -> optional RMSNorm (qw6_cpu_rmsnorm, qw6.c:2503-2513) ->
// router logits; one wave per expert row. Each wave holds the whole input
// in registers, so with norm_w set every wave computes the norm scale itself
// and wave e writes its slice of the normalised input for the expert kernels.
// Block n_experts (when present) computes the shared-expert gate weight
// sigmoid(shared_router . x) (qw6.c:2267-2285). NV = hidden / 256 float4 per
// lane, a template constant so that every load is unconditional. With a.xa
// set, waves e < hidden / 32 also write the small-batch MFMA operands.
// MT: one token per row of the grid (blockIdx.y; T = 1), as the expert
// kernels' launches of several tokens; the grid's x extent is rounded up to a
// multiple of 8, so router row e is read on XCD e % 8 for every token.
template <int T, int NV, bool MT = false>
__global__ __launch_bounds__(64) void k_moe_router(MoeArgs a) {
    TRACE_SCOPE(0);
    const uint32_t lane = threadIdx.x, e = blockIdx.x;
    const uint32_t H = 256 * NV;   // NV float4 per lane
    if constexpr (MT) {
        static_assert(T == 1, "one token per grid row");
        if (e >= a.n_experts + (a.shared_router ? 1u : 0u)) return;   // the rounding's workgroups
        const uint32_t t = blockIdx.y;
        a.x += (size_t)t * H;
        a.xn += (size_t)t * H;
        a.logits += (size_t)t * a.n_experts;
        a.sw += t;
    }
    float4 xv[T][NV];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (uint32_t i = 0; i < NV; i++)
            xv[t][i] = ((const float4*)(a.x + (size_t)t * H))[64 * i + lane];
    // the router row of expert e (or the shared-expert router); none when the
    // logits are given and this launch only normalises the input
    const float* wrow = e < a.n_experts ? a.router : e == a.n_experts ? a.shared_router : nullptr;
    if (wrow && e < a.n_experts) wrow += (size_t)e * H;
    float4 wv[NV];
#pragma unroll
    for (uint32_t i = 0; i < NV; i++)
        if (wrow) wv[i] = ((const float4*)wrow)[64 * i + lane];
    float sc_l = 1.0f;   // the RMSNorm scale of token (lane % 16) / 4 (operand row)
    if (a.norm_w) {
        float4 nw[NV];
#pragma unroll
        for (uint32_t i = 0; i < NV; i++)
            nw[i] = ((const float4*)a.norm_w)[64 * i + lane];
#pragma unroll
        for (int t = 0; t < T; t++) {
            float ss = 0.f;
#pragma unroll
            for (uint32_t i = 0; i < NV; i++) {
                ss = fmaf(xv[t][i].x, xv[t][i].x, ss); ss = fmaf(xv[t][i].y, xv[t][i].y, ss);
                ss = fmaf(xv[t][i].z, xv[t][i].z, ss); ss = fmaf(xv[t][i].w, xv[t][i].w, ss);
            }
            ss = group_sum<64>(ss);
            const float sc = 1.0f / sqrtf(ss / (float)H + a.norm_eps);
            if ((uint32_t)t == (lane & 15u) >> 2) sc_l = sc;
#pragma unroll
            for (uint32_t i = 0; i < NV; i++) {
                xv[t][i].x = xv[t][i].x * sc * nw[i].x; xv[t][i].y = xv[t][i].y * sc * nw[i].y;
                xv[t][i].z = xv[t][i].z * sc * nw[i].z; xv[t][i].w = xv[t][i].w * sc * nw[i].w;
            }
            // wave e writes float4s [e * per, (e + 1) * per) of the normalised input
            const uint32_t nq = H / 4, nwv = a.n_experts + (a.shared_router ? 1u : 0u);
            const uint32_t per = (nq + nwv - 1) / nwv;
#pragma unroll
            for (uint32_t i = 0; i < NV; i++) {
                const uint32_t q = 64 * i + lane;
                if (q >= e * per && q < (e + 1) * per)
                    ((float4*)(a.xn + (size_t)t * H))[q] = xv[t][i];
            }
        }
    }
    if (a.xa && e < H / 32) mx_input_operands<T>(a, e, sc_l);
    if (!wrow) return;
#pragma unroll
    for (int t = 0; t < T; t++) {
        float acc = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < NV; i++) {
            acc = fmaf(wv[i].x, xv[t][i].x, acc); acc = fmaf(wv[i].y, xv[t][i].y, acc);
            acc = fmaf(wv[i].z, xv[t][i].z, acc); acc = fmaf(wv[i].w, xv[t][i].w, acc);
        }
        acc = group_sum<64>(acc);
        if (lane == 0) {
            if (e < a.n_experts) a.logits[(size_t)t * a.n_experts + e] = acc;
            else a.sw[t] = 1.0f / (1.0f + expf(-acc));
        }
    }
}

// k_moe_router for one token on W waves per router row: wave h takes the
// float4 columns [h NV/W, (h + 1) NV/W) of the row, the input and the norm
// weight; the parts' sums (of squares for the norm, of products for the
// logit) meet in LDS and are added in wave order.
// MT: one token per row of the grid (blockIdx.y), the grid's x extent a
// multiple of 8, as k_moe_router<1, NV, true>.
template <int NV, int W, bool MT = false>
__global__ __launch_bounds__(64 * W) void k_moe_router_w(MoeArgs a) {
    constexpr int NH = NV / W;   // float4 per lane per wave
    static_assert(NH >= 1 && NH * W == NV, "W divides the row's float4 per lane");
    __shared__ float s_part[2][W];   // [sum of squares, dot product][wave]
    const uint32_t lane = threadIdx.x & 63u, h = threadIdx.x >> 6, e = blockIdx.x;
    const uint32_t H = 256 * NV;
    if constexpr (MT) {
        if (e >= a.n_experts + (a.shared_router ? 1u : 0u)) return;   // the rounding's workgroups
        const uint32_t t = blockIdx.y;
        a.x += (size_t)t * H;
        a.xn += (size_t)t * H;
        a.logits += (size_t)t * a.n_experts;
        a.sw += t;
    }
    float4 xv[NH];
#pragma unroll
    for (int i = 0; i < NH; i++) xv[i] = ((const float4*)a.x)[64 * (h * NH + i) + lane];
    const float* wrow = e < a.n_experts ? a.router : e == a.n_experts ? a.shared_router : nullptr;
    if (wrow && e < a.n_experts) wrow += (size_t)e * H;
    float4 wv[NH];
#pragma unroll
    for (int i = 0; i < NH; i++)
        if (wrow) wv[i] = ((const float4*)wrow)[64 * (h * NH + i) + lane];
    if (a.norm_w) {
        float4 nw[NH];
#pragma unroll
        for (int i = 0; i < NH; i++) nw[i] = ((const float4*)a.norm_w)[64 * (h * NH + i) + lane];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NH; i++) {
            ss = fmaf(xv[i].x, xv[i].x, ss); ss = fmaf(xv[i].y, xv[i].y, ss);
            ss = fmaf(xv[i].z, xv[i].z, ss); ss = fmaf(xv[i].w, xv[i].w, ss);
        }
        ss = group_sum<64>(ss);
        if (lane == 0) s_part[0][h] = ss;
        __syncthreads();
        float sst = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) sst += s_part[0][w];
        const float sc = 1.0f / sqrtf(sst / (float)H + a.norm_eps);
        const uint32_t nq = H / 4, nwv = a.n_experts + (a.shared_router ? 1u : 0u);
        const uint32_t per = (nq + nwv - 1) / nwv;
#pragma unroll
        for (int i = 0; i < NH; i++) {
            xv[i].x = xv[i].x * sc * nw[i].x; xv[i].y = xv[i].y * sc * nw[i].y;
            xv[i].z = xv[i].z * sc * nw[i].z; xv[i].w = xv[i].w * sc * nw[i].w;
            const uint32_t q = 64 * (h * NH + i) + lane;
            if (q >= e * per && q < (e + 1) * per) ((float4*)a.xn)[q] = xv[i];
        }
    }
    if (!wrow) return;   // the same for every wave
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NH; i++) {
        acc = fmaf(wv[i].x, xv[i].x, acc); acc = fmaf(wv[i].y, xv[i].y, acc);
        acc = fmaf(wv[i].z, xv[i].z, acc); acc = fmaf(wv[i].w, xv[i].w, acc);
    }
    acc = group_sum<64>(acc);
    if (lane == 0) s_part[1][h] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) v += s_part[1][w];
        if (e < a.n_experts) a.logits[e] = v;
        else a.sw[0] = 1.0f / (1.0f + expf(-v));
    }
}

// gate/up/silu of one wave: S steps of rps rows starting at row0 of the pair
// (G, Up) -> mid[T][inter]. slots: S LDS pair slots of pb bytes. x: the T
// input rows (hidden values each); this lane's activations are requested
// just before the weights, so both round trips overlap. bar: wait for the
// block's earlier LDS-direct loads (the lattice tables) and meet the other
// waves before reading them.
template <int T, int FF, int KU, int S = kStepsGu, bool LATE = false>
__device__ __forceinline__ void wave_gate_up(const MatD& G, const MatD& Up, uint32_t row0,
                                             const float* x, uint32_t hidden, bool bar,
                                             float* mid, uint32_t inter, uint8_t* slots,
                                             const uint32_t* lds, uint32_t slot_off, uint32_t pb,
                                             const uint32_t* tab) {
    const int f = FF >= 0 ? FF : G.fmt;
    constexpr uint32_t U = KU, rps = 64 / KU;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t unit = lane & (U - 1), blk = unit >> 3, q = lane / U;
    const int j = (int)(unit & 7);
    const uint32_t bb = fmt_block_bytes(f);
    const uint32_t gbytes = rps * G.rb;   // one step group (8 blocks)
    const uint32_t nl = FF >= 0 ? pair_loads(FF) : pair_loads(f);
    float xr[T][32];
    load_x_all<T, FF>(f, x, hidden, hidden, xr);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const size_t r = row0 + (size_t)s * rps;
        stage_pair(slots + s * pb, G.p + r * G.rb, Up.p + r * Up.rb, gbytes, nl);
    }
    TRACE_MARK(2, 5);
    // nothing that reads the activations may be scheduled among the staging
    // loads (its wait would hold back the loads after it)
    __builtin_amdgcn_sched_barrier(0);
    // LATE: a body that reads no lattice table (a K-quant format) meets the
    // other waves after its products instead: its own table loads are older
    // than its weights, so they have landed by then, and it computes while
    // the routed IQ waves wait for their weights. (The launches of several
    // tokens, two or three workgroups per CU, keep the barrier first:
    // measured slower there.)
    constexpr bool late_bar = LATE && FF >= 0 && !is_iq(FF);
    if (bar && !late_bar) {   // the block's earlier LDS-direct loads (the tables) are complete
        wait_vm(nl * S + 8u * T);
        lds_barrier();
    }
    const uint32_t boff = slot_off + q * G.rb + blk * bb;
    float sx[T][4];
    float ag[T][S], au[T][S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        wait_vm(nl * (S - 1 - s));
        TRACE_MARK_IF(s == 0, 2, 1);
        if (s == 0) x_sums_all<T>(f, xr, sx);   // the activations landed before step 0's weights
        float g[T], u[T];
#pragma unroll
        for (int t = 0; t < T; t++) { g[t] = 0.f; u[t] = 0.f; }
        unit_dot<T>(f, lds, s * pb + boff, j, tab, xr, sx, g);
        unit_dot<T>(f, lds, s * pb + gbytes + boff, j, tab, xr, sx, u);
#pragma unroll
        for (int t = 0; t < T; t++) { ag[t][s] = g[t]; au[t][s] = u[t]; }
    }
    TRACE_MARK(2, 2);
    float gv[T], uv[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
        gv[t] = reduce_scatter_k<S, KU>(ag[t]);
        uv[t] = reduce_scatter_k<S, KU>(au[t]);
    }
    if ((unit & (U / S - 1)) == 0) {
        const uint32_t s = scatter_step<S>(lane, U);
        const uint32_t r = row0 + s * rps + q;
#pragma unroll
        for (int t = 0; t < T; t++)
            mid[(size_t)t * inter + r] = gv[t] / (1.0f + expf(-gv[t])) * uv[t];
    }
    if (bar && late_bar) lds_barrier();
    TRACE_MARK(2, 3);
}

// One token, every gate/up pair of the layer in each workgroup: workgroup b
// takes rows [b R, (b + 1) R) (R = 2 rps, two row steps) of every selected
// expert and of the shared one. Wave w < top_k works on the expert of rank w
// (slot w), which it selects itself from the logits (no barrier); in
// workgroup 0, wave 0 runs the full routing instead and publishes the
// selection and the slot table. The waves past top_k (when the layer has a
// shared expert) stream the shared expert from the start (its waves:
// gate_up1_shared_waves). Every workgroup moves the same bytes and there is
// one per row tile: at hidden 2048 / inter 512, 256 workgroups of 9 or 10
// waves, one per CU (a 4-wave workgroup per (expert, row tile) put 576
// workgroups on the 256 CUs, three on a quarter of them).
//
// The shared expert takes two waves of one row step each for one token on
// layers whose gate/up formats include an IQ one: with nine waves one SIMD
// ran two routed waves and the whole shared expert, and the IQ units' decode
// made it the last to finish. K-quant layers, and the launches of several
// tokens (MT), whose workgroups share a CU two or three at a time, keep one
// wave of both row steps.
__host__ __device__ constexpr uint32_t gate_up1_shared_waves(bool mt, int fg) {
    return !mt && (fmt_in(fg, F_IQ2XXS) || fmt_in(fg, F_IQ2S) || fmt_in(fg, F_IQ3S)) ? 2u : 1u;
}

template <int FG, int KU, bool MT = false>
__global__ __launch_bounds__(64 * (8 + gate_up1_shared_waves(MT, FG))) void k_moe_gate_up1(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ uint32_t s_idx[8];
    __shared__ float s_w[8];
    __shared__ uint2 s_route[8 * kRouteScr];   // one per routed wave
    constexpr int S = kStepsGu;
    constexpr int SS = S / (int)gate_up1_shared_waves(MT, FG);   // row steps of a shared wave
    static_assert(SS * (int)gate_up1_shared_waves(MT, FG) == S, "the shared waves split the row steps");
    constexpr uint32_t rps = 64 / KU;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if constexpr (MT) token_view(a);
    const bool shared_w = wave >= a.top_k;
    const uint32_t sh_i = shared_w ? wave - a.top_k : 0u;   // a shared wave's share of the steps
    const uint32_t toff = tab_bytes(a.tmask_gu);
    // LDS pair slots: S per routed wave, then SS per shared wave
    const uint32_t slot_off = toff + (shared_w ? S * a.top_k + SS * sh_i : S * wave) * a.gu_pb;
    // the logits load is a routed wave's first memory operation; every wave
    // then stages its share of the lattice tables
    uint32_t keys[4];
    if (!shared_w) route_keys(a.route_logits, a.n_experts, keys);
    stage_tables_from(smem, a.tmask_gu, 0);
    const bool bar = a.tmask_gu != 0;   // wave_gate_up waits for them, then meets the others
    MatD G, Up;
    float* midp;
    if (shared_w) {
        G = a.sg;
        Up = a.su;
        midp = a.mid + (size_t)a.max_u * a.inter;
    } else {
        uint32_t e;
        if (blockIdx.x == 0 && wave == 0) {
            // publish the routing and the slot table for k_moe_down (one
            // token: the slots are the selection itself)
            wave_route_keys(keys, a.top_k, s_route, s_idx, s_w);
            __builtin_amdgcn_wave_barrier();
            if (lane < a.top_k) {
                const uint32_t o = (MT ? blockIdx.y * a.top_k : 0u) + lane;   // token_view's token
                if (a.idx_out) a.idx_out[o] = s_idx[lane];
                if (a.w_out) a.w_out[o] = s_w[lane];
                SlotTable* st = a.slots;
                const MatD D = expert_mat(a, s_idx[lane], 2);
                st->p[lane] = D.p; st->fmt[lane] = D.fmt; st->rb[lane] = D.rb;
                st->wt[lane][0] = s_w[lane];
#pragma unroll
                for (uint32_t t = 1; t < kMaxTok; t++) st->wt[lane][t] = 0.f;
            }
            if (lane == 0) a.slots->n = a.top_k;
            e = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_idx[0]);
        } else {
            e = wave_route_select(keys, a.top_k, wave, s_route + wave * kRouteScr);
        }
        G = expert_mat_wave(a, e, 0);
        Up = expert_mat_wave(a, e, 1);
        midp = a.mid + (size_t)wave * a.inter;
    }
    const uint32_t row0 = (blockIdx.x * S + sh_i * SS) * rps;
    const uint32_t* lds = (const uint32_t*)smem;
    uint8_t* wslots = smem + slot_off;
    auto body = [&](auto fc) {
        constexpr int F = decltype(fc)::value;
        if constexpr (SS == S) {
            wave_gate_up<1, F, KU, S, !MT>(G, Up, row0, a.xin, a.hidden, bar, midp, a.inter, wslots, lds,
                                           slot_off, a.gu_pb, lds);
        } else if (shared_w) {
            wave_gate_up<1, F, KU, SS, !MT>(G, Up, row0, a.xin, a.hidden, bar, midp, a.inter, wslots, lds,
                                            slot_off, a.gu_pb, lds);
        } else {
            wave_gate_up<1, F, KU, S, !MT>(G, Up, row0, a.xin, a.hidden, bar, midp, a.inter, wslots, lds,
                                           slot_off, a.gu_pb, lds);
        }
    };
    if constexpr (FG >= 0) {
        body(std::integral_constant<int, FG>{});
    } else {   // mixed formats: one switch per wave, each body specialised
        by_fmt<FG>(G.fmt, body);
    }
}

// Down projection + combine for rows [r0, r0 + R), R = S * rps. Matrix m of
// the block: m = 0 the shared expert (when present; no routing needed, so
// its wave starts streaming at once), then the slots in first-use order.
// Wave w takes matrices w, w + nw, ...; row sums meet in LDS and are
// combined as out = sum_u wt[u] * y[u] + sw * y[shared] (+ residual).
// (9: the 8 routed matrices of a token and the shared one)
template <int T>
__host__ __device__ constexpr uint32_t down_waves() { return T <= 2 ? 9u : 8u; }

// The kStepsDn row steps of one down matrix staged in LDS, the lane's row at
// byte offset boff0: per-lane unit dot products, reduced over the row's
// lanes; ym[rl * T + t] = row rl's sum for token t.
template <int T, int F, int KU>
__device__ __forceinline__ void down_rows(const uint32_t* lds, uint32_t boff0, int j,
                                          const float (&xr)[T][32], float* ym) {
    constexpr int S = kStepsDn;
    constexpr uint32_t U = KU, rps = 64 / KU;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t unit = lane & (U - 1), q = lane / U;
    const uint32_t boff = boff0 + (unit >> 3) * fmt_block_bytes(F);
    float sx[T][4];
    x_sums_all<T>(F, xr, sx);
    float acc[T][S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        wait_vm(2u * (S - 1 - s));
        float v[T];
#pragma unroll
        for (int t = 0; t < T; t++) v[t] = 0.f;
        unit_dot<T>(F, lds, s * kSlotBytes + boff, j, lds, xr, sx, v);
#pragma unroll
        for (int t = 0; t < T; t++) acc[t][s] = v[t];
    }
    float r[T];
#pragma unroll
    for (int t = 0; t < T; t++) r[t] = reduce_scatter_k<S, KU>(acc[t]);
    if ((unit & (U / S - 1)) == 0) {
        const uint32_t rl = scatter_step<S>(lane, U) * rps + q;
#pragma unroll
        for (int t = 0; t < T; t++) ym[rl * T + t] = r[t];
    }
}

template <int T, int FD, int KU, bool MT = false>
__global__ __launch_bounds__(64 * down_waves<T>()) void k_moe_down(MoeArgs a) {
    TRACE_SCOPE(3);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float s_wt[kMaxSlots * kMaxTok];
    constexpr int S = kStepsDn;
    constexpr uint32_t U = KU, rps = 64 / KU;
    constexpr uint32_t R = S * rps;
    static_assert(!MT || T == 1, "launches over several tokens run the one-token kernel");
    if constexpr (MT) token_view(a);
    const uint32_t r0 = blockIdx.x * R;
    const uint32_t nw = blockDim.x >> 6;
    // wave index as a wave-uniform value: the slot-table reads below then
    // become scalar loads
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t has_sh = a.sd.p != nullptr ? 1u : 0u;
    // The slot table is read in one round trip: the count and this wave's
    // first slot (speculatively: entries past the count repeat slot 0) are scalar
    // loads issued before anything else. Issued after the lattice tables'
    // LDS-direct loads they would be vector loads whose use waits for every
    // earlier vector load (the counter retires in order). The gate weights,
    // the combine's residual and shared weight are fetched now too.
    const uint32_t nslot = a.slots->n;
    const uint32_t u0 = wave - has_sh;
    const bool first_sh = has_sh && wave == 0;
    const uint32_t u0c = first_sh ? 0u : min(u0, kMaxSlots - 1);
    const uint8_t* p0 = a.slots->p[u0c];
    const int f0 = a.slots->fmt[u0c];
    const uint32_t rb0 = a.slots->rb[u0c];
    const uint32_t toff = tab_bytes(a.tmask_dn);
    stage_tables(smem, a.tmask_dn);
    float* ybuf = (float*)(smem + toff + nw * S * kSlotBytes);   // [m][R][T]
    uint8_t* slots = smem + toff + wave * S * kSlotBytes;
    const uint32_t slot_off = toff + wave * S * kSlotBytes;
    const uint32_t unit = lane & (U - 1), q = lane / U;
    const int j = (int)(unit & 7);
    // (the gate weights go to LDS only after the products: an LDS write here
    // would wait for every vector load issued before it)
    const float wt_l = threadIdx.x < kMaxSlots * kMaxTok
                           ? a.slots->wt[threadIdx.x / kMaxTok][threadIdx.x % kMaxTok] : 0.f;
    float resid = 0.f, shw = 1.0f;
    if (threadIdx.x < R * T) {
        const uint32_t rl = threadIdx.x / T, t = threadIdx.x % T;
        if (a.residual) resid = a.residual[((size_t)t + (MT ? blockIdx.y : 0u)) * a.hidden + r0 + rl];
        if (has_sh && a.shared_router) shw = a.sw[t];
    }
    const uint32_t ntot = nslot + has_sh;
    // One matrix of this wave. The first is peeled off the loop below: every
    // wave takes one and issues its loads before the barrier that makes the
    // lattice tables visible, and a loop around it (or a branch on the
    // count) would make the compiler wait for earlier loads (the gate
    // weights, residual, lattice tables, the count) before its activation
    // loads. The launch has nw <= max_u + has_sh waves, and k_moe_gate_up1
    // publishes every rank of its token (n = max_u = top_k), so each wave's
    // first matrix is a selected one. (A table's entries past its count
    // repeat slot 0's matrix: a wave past the count would stream real
    // weights into a ybuf row the combine does not read, m < nw keeping
    // the row inside the allocation.)
    auto matrix = [&](uint32_t m, bool first) {
        const bool sh = has_sh && m == 0;
        const uint32_t u = m - has_sh;
        const float* xm = a.mid + (size_t)(sh ? a.max_u : u) * T * a.inter;
        float xr[T][32];
        // activations before the slot table's answer when their layout is
        // known already (one format, the shared expert, or one layout class)
        const int fx = FD >= 0 ? FD : sh ? a.sd.fmt : a.xl_dn;
        if (fx >= 0) load_x_all<T, FD>(fx, xm, a.inter, a.inter, xr);
        const MatD D = sh ? a.sd
                          : first ? MatD{p0, f0, a.hidden, a.inter, rb0}
                                  : MatD{a.slots->p[u], a.slots->fmt[u], a.hidden, a.inter,
                                         a.slots->rb[u]};
        const int f = FD >= 0 ? FD : D.fmt;
        if (fx < 0) load_x_all<T, FD>(f, xm, a.inter, a.inter, xr);
#pragma unroll
        for (int s = 0; s < S; s++)
            stage_group(slots + s * kSlotBytes, D.p + (size_t)(r0 + s * rps) * D.rb, rps * D.rb);
        TRACE_MARK_IF(first, 3, 0);
        if (a.tmask_dn && first) {
            wait_vm(8u * T + 2u * S);   // this wave's table loads (its oldest) have landed
            lds_barrier();              // and every other wave's: the tables are complete
        }
        const uint32_t boff = slot_off + q * D.rb;   // the lane's row; + its block below
        float* ym = ybuf + m * R * T;
        if (FD >= 0) {
            down_rows<T, FD, KU>((const uint32_t*)smem, boff, j, xr, ym);
        } else {   // mixed formats: one switch per matrix, each body specialised
            by_fmt<FD>(f, [&](auto fc) {
                down_rows<T, decltype(fc)::value, KU>((const uint32_t*)smem, boff, j, xr, ym);
            });
        }
        TRACE_MARK_IF(first, 3, 1);
    };
    matrix(wave, true);
    for (uint32_t m = wave + nw; m < ntot; m += nw) matrix(m, false);
    TRACE_MARK(3, 2);
    if (threadIdx.x < kMaxSlots * kMaxTok) s_wt[threadIdx.x] = wt_l;
    __syncthreads();
    static_assert(R * T <= 64, "one combine output per thread of the smallest block");
    if (threadIdx.x < R * T) {
        const uint32_t rl = threadIdx.x / T, t = threadIdx.x % T;
        float v = 0.f;
        for (uint32_t u = 0; u < nslot; u++)
            v = fmaf(s_wt[u * kMaxTok + t], ybuf[((u + has_sh) * R + rl) * T + t], v);
        if (has_sh) v = fmaf(shw, ybuf[rl * T + t], v);
        if (a.residual) v += resid;
        a.out[(size_t)t * a.hidden + r0 + rl] = v;
    }
}

// ---- small-batch MFMA kernels ------------------------------------------------------
// k_mx_gate_up and k_mx_down compute the same layer as k_moe_gate_up1 and
// k_moe_down for T <= 4 tokens, with bf16 MFMA 16x16x32 on the operands above:
// the weights' per-lane decode work (qw6_tile.h) no longer grows with T, and
// the registers no longer hold every token's activations.

// LDS of the bf16 lattice grids of the IQ formats in a fmt_table_mask, the
// grids present in the order IQ2_XXS, IQ2_S, IQ3_S (signs are computed).
struct MxTab {
    uint32_t g[3];
    uint32_t bytes;
};
__host__ __device__ inline MxTab mx_tab(uint32_t mask) {
    MxTab t;
    uint32_t o = 0u;
    const uint32_t gb[3] = {256u * 16u, 1024u * 16u, 512u * 8u};
    for (int i = 0; i < 3; i++) {
        t.g[i] = o;
        if ((mask >> i) & 1u) o += gb[i];
    }
    t.bytes = o;
    return t;
}
__device__ __forceinline__ void stage_mx_tables(uint8_t* tab, uint32_t mask, uint32_t nthr) {
    if (!mask) return;
    const MxTab tb = mx_tab(mask);
    if (mask & 1u) stage_iq_grid<F_IQ2XXS>(tab + tb.g[0], g_tabs, nthr);
    if (mask & 2u) stage_iq_grid<F_IQ2S>(tab + tb.g[1], g_tabs, nthr);
    if (mask & 4u) stage_iq_grid<F_IQ3S>(tab + tb.g[2], g_tabs, nthr);
}

// 16-byte loads per lane that stage one 256-column block of 16 rows.
__host__ __device__ constexpr uint32_t mx_stage_loads(int f) { return (16u * raw_chunks(f) + 63u) / 64u; }
__host__ __device__ constexpr uint32_t mx_stage_bytes(int f) { return 1024u * mx_stage_loads(f); }

// Stage the block at byte offset boff of 16 rows (row r at src + r * rb) into
// LDS dst (one wave): row r's chunk k (16 B from the line that holds the
// block's start) lands at dst + 16 (r * raw_chunks(f) + k). Chunks past a row's
// block reload its first chunk, so no load reaches past the block's last line.
__device__ __forceinline__ void mx_stage(uint8_t* dst, const uint8_t* src, uint32_t rb, uint32_t boff,
                                         int f) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nch = raw_chunks(f), bb = fmt_block_bytes(f), nl = mx_stage_loads(f);
    for (uint32_t i = 0; i < nl; i++) {
        const uint32_t c = 64u * i + lane;
        const bool in = c < 16u * nch;
        const uint32_t r = in ? c / nch : 0u, k = in ? c % nch : 0u;
        const uint8_t* p = src + (size_t)r * rb + boff;
        const uint32_t off = (uint32_t)((uintptr_t)p & 15u);
        const uint32_t kk = 16u * k < off + bb ? k : 0u;
        __builtin_amdgcn_global_load_lds((glb_void_t*)(p - off + 16u * kk), (lds_void_t*)(dst + 1024u * i),
                                         16, 0, 0);
    }
}
// LDS byte offset of row n's block staged by mx_stage at LDS offset so.
__device__ __forceinline__ uint32_t mx_row_off(uint32_t so, const uint8_t* src, uint32_t rb, uint32_t boff,
                                               uint32_t n, int f) {
    return so + 16u * raw_chunks(f) * n + (uint32_t)((uintptr_t)(src + (size_t)n * rb + boff) & 15u);
}

// A operands of block kb: sub-block entries 8 kb .. 8 kb + 7 of ea, and the
// half-sum operands of es in lanes m = 4 t (k-slots 8 q + j, q < 3).
__device__ __forceinline__ void mx_load_a(const uint4* ea, const uint16_t* es, uint32_t kb, uint32_t lane,
                                          uint4 (&av)[8], uint4& c0, uint4& c1) {
#pragma unroll
    for (int j = 0; j < 8; j++) av[j] = ea[(size_t)(8 * kb + j) * 64 + lane];
    const uint32_t m = lane & 15u, q = lane >> 4;
    c0 = make_uint4(0, 0, 0, 0);
    c1 = c0;
    if ((m & 3u) == 0 && q < 3) {
        const uint16_t* b = es + (((size_t)kb * 2) * 4 + (m >> 2)) * 24 + 8 * q;
        c0 = *(const uint4*)b;
        c1 = *(const uint4*)(b + 4 * 24);
    }
}

// mx_block for the runtime format f (uniform across the wave).
__device__ __forceinline__ void mx_block_fmt(int f, const uint32_t* s, const uint8_t* tab, const MxTab& tb,
                                             uint32_t R, uint32_t q, const uint4 (&av)[8], const uint4& c0,
                                             const uint4& c1, f32x4& acc) {
    switch (f) {
    case F_Q4K: mx_block<F_Q4K>(s, tab, R, q, av, c0, c1, acc); break;
    case F_Q5K: mx_block<F_Q5K>(s, tab, R, q, av, c0, c1, acc); break;
    case F_Q6K: mx_block<F_Q6K>(s, tab, R, q, av, c0, c1, acc); break;
    case F_IQ2XXS: mx_block<F_IQ2XXS>(s, tab + tb.g[0], R, q, av, c0, c1, acc); break;
    case F_IQ2S: mx_block<F_IQ2S>(s, tab + tb.g[1], R, q, av, c0, c1, acc); break;
    default: mx_block<F_IQ3S>(s, tab + tb.g[2], R, q, av, c0, c1, acc); break;
    }
}

// Routing of one routed block of a gate/up kernel (tiles per slot: ntile):
// its slot u and tile, the slot's expert e, and for the first routed block the
// published selection and slot table. False: unused slot.
template <int T>
__device__ __forceinline__ bool mx_route_block(const MoeArgs& a, uint32_t (&keys)[4], uint32_t ntile,
                                               uint32_t& u, uint32_t& tile, uint32_t& e) {
    __shared__ uint32_t s_idx[kMaxSlots], s_slot_e[kMaxSlots], s_n;
    __shared__ float s_w[kMaxSlots], s_wt[kMaxSlots * kMaxTok];
    __shared__ uint2 s_route[T * kRouteScr];
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t b = blockIdx.x - a.n_sh_wg;
    u = b / ntile;
    tile = b % ntile;
    if (T == 1 && b != 0) {   // one token: only the expert of rank u
        if (wave == 0) {
            const uint32_t x = wave_route_select(keys, a.top_k, u, s_route);
            if ((threadIdx.x & 63u) == 0) s_n = x;
        }
        __syncthreads();
        e = s_n;
        return true;
    }
    if (b != 0) return route_slot_select<T>(a, keys, u, e, s_route, s_idx);
    route_prologue<T>(a, keys, s_route, s_idx, s_w, s_slot_e, s_wt, &s_n);   // ends with a barrier
    const uint32_t nslot = s_n;
    if (b == 0) {
        const uint32_t tid = threadIdx.x;
        if (tid < T * a.top_k) {
            if (a.idx_out) a.idx_out[tid] = s_idx[tid];
            if (a.w_out) a.w_out[tid] = s_w[tid];
        }
        if (tid < a.max_u) {
            SlotTable* st = a.slots;
            // entries past the count name slot 0's matrix (weight 0 for every
            // token): each k_moe_down wave stages its first matrix before it
            // knows the count, so every entry a wave may take must be a real
            // matrix (nslot >= 1: top_k >= 1)
            const MatD D = expert_mat(a, s_slot_e[tid < nslot ? tid : 0u], 2);
            st->p[tid] = D.p; st->fmt[tid] = D.fmt; st->rb[tid] = D.rb;
#pragma unroll
            for (uint32_t t = 0; t < kMaxTok; t++) st->wt[tid][t] = s_wt[tid * kMaxTok + t];
        }
        if (tid == 0) a.slots->n = nslot;
    }
    if (u >= nslot) return false;
    e = s_slot_e[u];
    return true;
}

// Gate / up of 16 intermediate rows [row0, row0 + 16) of one matrix pair, all
// waves: wave w takes the 256-column blocks w, w + nw, ...; their (gate, up)
// bytes are staged at once. Leaves this lane's D sums in ag / au.
template <int FW>
__device__ __forceinline__ void mx_gu_blocks(const MoeArgs& a, const MatD& Gm, const MatD& Um, uint32_t row0,
                                             uint8_t* smem, uint32_t soff, const MxTab& tb, f32x4& ag,
                                             f32x4& au) {
    uint4 av[8], c0, c1;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, nw = blockDim.x >> 6;
    const uint32_t n = lane & 15u, q = lane >> 4;
    const uint32_t nkb = a.hidden / 256, nbw = (nkb + nw - 1) / nw;
    constexpr uint32_t SB = mx_stage_bytes(FW), bb = fmt_block_bytes(FW);
    const uint32_t so = soff + wave * nbw * 2 * SB;
    const uint8_t* g0 = Gm.p + (size_t)row0 * Gm.rb;
    const uint8_t* u0 = Um.p + (size_t)row0 * Um.rb;
    for (uint32_t i = 0, kb = wave; kb < nkb; i++, kb += nw) {
        mx_stage(smem + so + 2 * i * SB, g0, Gm.rb, kb * bb, FW);
        mx_stage(smem + so + (2 * i + 1) * SB, u0, Um.rb, kb * bb, FW);
    }
    for (uint32_t i = 0, kb = wave; kb < nkb; i++, kb += nw) {
        mx_load_a(a.xa, a.xs, kb, lane, av, c0, c1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        TRACE_MARK_IF(i == 0, 2, 1);
        const uint32_t Rg = mx_row_off(so + 2 * i * SB, g0, Gm.rb, kb * bb, n, FW);
        const uint32_t Ru = mx_row_off(so + (2 * i + 1) * SB, u0, Um.rb, kb * bb, n, FW);
        const uint8_t* grid = smem + tb.g[FW >= F_IQ2XXS ? FW - F_IQ2XXS : 0];
        mx_block<FW>((const uint32_t*)smem, grid, Rg, q, av, c0, c1, ag);
        __builtin_amdgcn_sched_barrier(0);   // gate then up: one block's temporaries live at a time
        mx_block<FW>((const uint32_t*)smem, grid, Ru, q, av, c0, c1, au);
    }
}

// Routed + shared gate/up/SiLU: block (matrix pair, 16-row tile), shared
// expert first (blocks [0, n_sh_wg)); writes the down kernel's operands of mid.
// Launched with at least kMaxTok waves: wave t routes token t.
template <int T>
__global__ __launch_bounds__(512, 4) void k_mx_gate_up(MoeArgs a) {
    TRACE_SCOPE(2);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float s_gu[2][kMaxTok][16];
    __shared__ float s_mid[kMaxTok][16];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u, nw = blockDim.x >> 6;
    const uint32_t ntile = a.inter / 16;
    const bool shared_wg = blockIdx.x < a.n_sh_wg;
    // routing waves load their logits first; every wave then loads the A
    // operands of its first block, which do not depend on the routing
    uint32_t keys[4];
    if (!shared_wg && wave < (uint32_t)T)
        route_keys(a.route_logits + (size_t)wave * a.n_experts, a.n_experts, keys);
    const uint32_t tmask = shared_wg ? fmt_table_mask(a.sg.fmt) : a.tmask_gu;
    const MxTab tb = mx_tab(tmask);
    stage_mx_tables(smem, tmask, blockDim.x);
    MatD Gm, Um;
    uint32_t row0, slot;
    if (shared_wg) {
        Gm = a.sg;
        Um = a.su;
        row0 = blockIdx.x * 16;
        slot = a.max_u;
        if (tmask) __syncthreads();   // the lattice tables are complete
    } else {
        uint32_t u, tile, e;
        if (!mx_route_block<T>(a, keys, ntile, u, tile, e)) return;   // (barriers inside)
        Gm = expert_mat(a, e, 0);
        Um = expert_mat(a, e, 1);
        row0 = tile * 16;
        slot = u;
    }
    TRACE_MARK(2, 0);
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
    const uint32_t soff = a.mx_gu_soff;   // staging after the largest table set
    switch (Gm.fmt) {
    case F_Q4K: mx_gu_blocks<F_Q4K>(a, Gm, Um, row0, smem, soff, tb, ag, au); break;
    case F_Q5K: mx_gu_blocks<F_Q5K>(a, Gm, Um, row0, smem, soff, tb, ag, au); break;
    case F_Q6K: mx_gu_blocks<F_Q6K>(a, Gm, Um, row0, smem, soff, tb, ag, au); break;
    case F_IQ2XXS: mx_gu_blocks<F_IQ2XXS>(a, Gm, Um, row0, smem, soff, tb, ag, au); break;
    case F_IQ2S: mx_gu_blocks<F_IQ2S>(a, Gm, Um, row0, smem, soff, tb, ag, au); break;
    default: mx_gu_blocks<F_IQ3S>(a, Gm, Um, row0, smem, soff, tb, ag, au); break;
    }
    TRACE_MARK(2, 2);
    // the waves' partial sums meet in LDS (over the staged bytes), fixed order
    __syncthreads();
    float* red = (float*)(smem + soff);   // [nw][2][64][4]
#pragma unroll
    for (int i = 0; i < 4; i++) {
        red[((wave * 2 + 0) * 64 + lane) * 4 + i] = ag[i];
        red[((wave * 2 + 1) * 64 + lane) * 4 + i] = au[i];
    }
    __syncthreads();
    if (tid < 128) {
        const uint32_t mat = tid >> 6, l = tid & 63u;
        float v = 0.f;
        for (uint32_t w = 0; w < nw; w++) {
            const float* r = red + ((w * 2 + mat) * 64 + l) * 4;
            v += (r[0] + r[1]) + r[2];
        }
        s_gu[mat][l >> 4][l & 15u] = v;
    }
    __syncthreads();
    if (tid < 64) {
        const uint32_t t = tid >> 4, nn = tid & 15u;
        float y = 0.f;
        if (t < (uint32_t)T) {
            const float g = s_gu[0][t][nn], u = s_gu[1][t][nn];
            y = g / (1.0f + expf(-g)) * u;
        }
        s_mid[t][nn] = y;
    }
    __syncthreads();
    // mid rows [row0, row0 + 16) are half h of sub-block sb of the down input
    const uint32_t sb = row0 >> 5, h = (row0 >> 4) & 1u;
    if (tid < 32) {
        const uint32_t qq = 2 * h + (tid >> 4), m = tid & 15u;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = s_mid[m >> 2][8 * (tid >> 4) + i];
        a.ma[((size_t)slot * (a.inter / 32) + sb) * 64 + 16 * qq + m] = mx_pack8(v, m & 3u);
    } else if (tid < 32 + kMaxTok) {
        const uint32_t t = tid - 32;
        float hs = 0.f;
        for (uint32_t nn = 0; nn < 16; nn++) hs += s_mid[t][nn];
        mx_put_halfsum(a.ms + (size_t)slot * (a.inter / 256) * 192, sb, h, t, hs);
    }
}

// Down projection + combine for hidden rows [r0, r0 + 16): the (matrix, block)
// pairs -- matrix 0 the shared expert when present, then the slots -- go to
// the waves in turn, staged a round of mx_nsl pairs at a time; per-pair sums
// meet in LDS and are combined as out = sum_u wt[u] * y[u] + sw * y[shared]
// (+ residual), a fixed order.
template <int T>
__global__ __launch_bounds__(1024) void k_mx_down(MoeArgs a) {
    TRACE_SCOPE(3);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float s_wt[kMaxSlots * kMaxTok];
    __shared__ const uint8_t* s_p[kMaxSlots];
    __shared__ int32_t s_fmt[kMaxSlots];
    __shared__ uint32_t s_rb[kMaxSlots];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u, nw = blockDim.x >> 6;
    const uint32_t n = lane & 15u, q = lane >> 4;
    const uint32_t r0 = blockIdx.x * 16;
    const uint32_t has_sh = a.sd.p != nullptr ? 1u : 0u;
    const uint32_t nkb = a.inter / 256;
    const MxTab tb = mx_tab(a.tmask_dn);
    // the slot table in one round trip (only entries below the count are used)
    const uint32_t nslot = a.slots->n;
    if (tid < kMaxSlots * kMaxTok) s_wt[tid] = a.slots->wt[tid / kMaxTok][tid % kMaxTok];
    if (tid < kMaxSlots) {
        s_p[tid] = a.slots->p[tid];
        s_fmt[tid] = a.slots->fmt[tid];
        s_rb[tid] = a.slots->rb[tid];
    }
    float resid = 0.f, shw = 1.0f;
    if (tid < 16 * T) {
        const uint32_t t = tid >> 4, nn = tid & 15u;
        if (a.residual) resid = a.residual[(size_t)t * a.hidden + r0 + nn];
        if (has_sh && a.shared_router) shw = a.sw[t];
    }
    stage_mx_tables(smem, a.tmask_dn, blockDim.x);
    __syncthreads();   // slot table and lattice tables
    TRACE_MARK(3, 0);
    const uint32_t ntot = nslot + has_sh, npair = ntot * nkb;
    const uint32_t soff = tb.bytes;
    float* ybuf = (float*)(smem + soff + a.mx_nsl * a.mx_sb);   // [pair][4][16]
    auto mat = [&](uint32_t m) -> MatD {
        if (has_sh && m == 0) return a.sd;
        const uint32_t u = m - has_sh;
        return MatD{s_p[u], s_fmt[u], a.hidden, a.inter, s_rb[u]};
    };
    for (uint32_t base = 0; base < npair; base += a.mx_nsl) {
        const uint32_t end = min(base + a.mx_nsl, npair);
        for (uint32_t pr = base + wave; pr < end; pr += nw) {
            const MatD D = mat(pr / nkb);
            const uint32_t kb = pr % nkb;
            mx_stage(smem + soff + (pr - base) * a.mx_sb, D.p + (size_t)r0 * D.rb, D.rb,
                     kb * fmt_block_bytes(D.fmt), D.fmt);
        }
        for (uint32_t pr = base + wave; pr < end; pr += nw) {
            const uint32_t m = pr / nkb, kb = pr % nkb;
            const bool sh = has_sh && m == 0;
            const MatD D = mat(m);
            const uint32_t slot = sh ? a.max_u : m - has_sh;
            uint4 av[8], c0, c1;
            mx_load_a(a.ma + (size_t)slot * (a.inter / 32) * 64, a.ms + (size_t)slot * nkb * 192, kb, lane,
                      av, c0, c1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            TRACE_MARK_IF(pr == wave, 3, 1);
            const uint32_t R = mx_row_off(soff + (pr - base) * a.mx_sb, D.p + (size_t)r0 * D.rb, D.rb,
                                          kb * fmt_block_bytes(D.fmt), n, D.fmt);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            mx_block_fmt(D.fmt, (const uint32_t*)smem, smem, tb, R, q, av, c0, c1, acc);
            ybuf[(pr * 4 + q) * 16 + n] = (acc[0] + acc[1]) + acc[2];
        }
        if (end < npair) __syncthreads();   // the next round reuses the staging slots
    }
    TRACE_MARK(3, 2);
    __syncthreads();
    if (tid < 16 * T) {
        const uint32_t t = tid >> 4, nn = tid & 15u;
        auto y = [&](uint32_t m) {
            float v = 0.f;
            for (uint32_t kb = 0; kb < nkb; kb++) v += ybuf[((m * nkb + kb) * 4 + t) * 16 + nn];
            return v;
        };
        float v = 0.f;
        for (uint32_t u = 0; u < nslot; u++) v = fmaf(s_wt[u * kMaxTok + t], y(u + has_sh), v);
        if (has_sh) v = fmaf(shw, y(0), v);
        if (a.residual) v += resid;
        a.out[(size_t)t * a.hidden + r0 + nn] = v;
    }
}

// ---- small elementwise kernels ---------------------------------------------------

__global__ void k_silu_mul(const float* g, const float* u, float* o, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

// ---- greedy argmax (qw6_cpu_argmax, qw6.c:2858-2863) ----------------------------
// qw6 scans i = 1 .. n-1 and keeps the first index whose value is strictly
// greater than the best so far: ties go to the lowest index, a NaN never
// wins, and a NaN at index 0 is never replaced (every comparison with it is
// false). Each value becomes the 64-bit key (order key of the value, ~index),
// a NaN the order key 0 (below -inf), so the largest key is the first maximum;
// the NaN-at-0 rule is applied at the end. The maximum is exact and
// associative: how the range is split over blocks cannot change the result.
constexpr uint32_t kArgmaxBlocks = 512;   // partial maxima of the first pass

__device__ __forceinline__ uint64_t amax_key(float v, uint32_t i) {
    const uint32_t k = v != v ? 0u : route_key(v, false);
    return ((uint64_t)k << 32) | (uint32_t)~i;
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
// Maximum over the 64 lanes of a wave; every lane receives it.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const uint32_t m = 32u >> i;
        const uint32_t lo = __float_as_uint(partner(__uint_as_float((uint32_t)v), m, lane));
        const uint32_t hi = __float_as_uint(partner(__uint_as_float((uint32_t)(v >> 32)), m, lane));
        v = max_u64(v, ((uint64_t)hi << 32) | lo);
    }
    return v;
}
// Maximum over a 256-thread block, returned to thread 0.
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* s4) {
    v = wave_max_u64(v);
    if ((threadIdx.x & 63u) == 0) s4[threadIdx.x >> 6] = v;
    __syncthreads();
    return max_u64(max_u64(s4[0], s4[1]), max_u64(s4[2], s4[3]));
}

// First pass: block b takes every gridDim.x-th float4 (then the tail).
__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ x, uint32_t n,
                                                     uint64_t* __restrict__ part) {
    __shared__ uint64_t s4[4];
    uint64_t best = 0;   // below every element's key (index 0xffffffff)
    const uint32_t t0 = blockIdx.x * 256 + threadIdx.x, stride = gridDim.x * 256;
    const uint32_t n4 = ((uintptr_t)x & 15u) ? 0u : n / 4;
    for (uint32_t i = t0; i < n4; i += stride) {
        const float4 v = ((const float4*)x)[i];
        best = max_u64(best, max_u64(max_u64(amax_key(v.x, 4 * i), amax_key(v.y, 4 * i + 1)),
                                     max_u64(amax_key(v.z, 4 * i + 2), amax_key(v.w, 4 * i + 3))));
    }
    for (uint32_t i = 4 * n4 + t0; i < n; i += stride) best = max_u64(best, amax_key(x[i], i));
    best = block_max_u64(best, s4);
    if (threadIdx.x == 0) part[blockIdx.x] = best;
}

// Second pass: one block over the nb partial maxima.
__global__ __launch_bounds__(256) void k_argmax_final(const float* __restrict__ x,
                                                      const uint64_t* __restrict__ part,
                                                      uint32_t nb, uint32_t* out) {
    __shared__ uint64_t s4[4];
    uint64_t best = 0;
    for (uint32_t i = threadIdx.x; i < nb; i += 256) best = max_u64(best, part[i]);
    best = block_max_u64(best, s4);
    if (threadIdx.x == 0) {
        const float x0 = x[0];
        out[0] = x0 != x0 ? 0u : ~(uint32_t)best;
    }
}

// ---- output head: one streaming pass over a large matrix ------------------------
// logits[r] = deq(W)[r] . (rmsnorm(x) * norm_w) for every row, plus each
// wave's running argmax key (part[wave]) for k_argmax_final. The layout of
// k_matvec (U = K/32 lanes per row, rps = 64/U rows per step), but each wave
// loads its activations once (the norm fused: a lane's 32 values of the
// first row group are the whole vector once) and streams its rows through
// kHeadSlots direct-to-LDS slots, so that many row steps are in flight.
// Step s of wave w covers row group w + s * (number of waves): neighbouring
// waves read neighbouring rows. Every wave issues the same loads: steps
// past the last row group restage group 0 and write nothing, so each wait
// is a constant; the wave drains its loads before it ends (an LDS-direct
// load must not land after the workgroup's LDS is released).
constexpr int kHeadSlots = 4;        // row steps in flight per wave
constexpr uint32_t kHeadWaves = 4096;   // waves of one launch, at most

template <int F, int KU>
__global__ __launch_bounds__(kWG) void k_head(const uint8_t* __restrict__ W, uint32_t groups,
                                              uint32_t rows, uint32_t rb, uint32_t nsteps,
                                              const float* __restrict__ x,
                                              const float* __restrict__ norm_w, float eps,
                                              float* __restrict__ logits,
                                              uint64_t* __restrict__ part, uint32_t tmask) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr uint32_t U = KU, rps = 64 / KU, K = 32 * KU;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t unit = lane & (U - 1), blk = unit >> 3, q = lane / U;
    const int j = (int)(unit & 7);
    const uint32_t gw = blockIdx.x * 4 + wave, nwv = gridDim.x * 4;
    const uint32_t soff = tab_bytes(tmask) + wave * kHeadSlots * kSlotBytes;
    const uint32_t gbytes = rps * rb;   // one row group: 8 GGUF blocks
    auto src = [&](uint32_t st) -> const uint8_t* {
        const uint32_t g = gw + st * nwv;
        return W + (size_t)(g < groups ? g : 0u) * gbytes;
    };
    stage_tables(smem, tmask);
#pragma unroll
    for (int st = 0; st < kHeadSlots; st++) stage_group(smem + soff + st * kSlotBytes, src(st), gbytes);
    float xr[1][32], sx[1][4];
    load_unit_x(F, x, blk, j, xr[0]);
    if (norm_w) {   // final RMSNorm (qw6.c:2490-2492)
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) ss = fmaf(xr[0][i], xr[0][i], ss);
        ss = group_sum<64>(q == 0 ? ss : 0.f);
        const float sc = 1.0f / sqrtf(ss / (float)K + eps);
        float wr[32];
        load_unit_x(F, norm_w, blk, j, wr);
#pragma unroll
        for (int i = 0; i < 32; i++) xr[0][i] = xr[0][i] * sc * wr[i];
    }
    unit_x_sums(F, xr[0], sx[0]);
    if (tmask) {   // the lattice tables (this wave's oldest loads) of every wave
        wait_vm(0);
        lds_barrier();
    }
    const uint32_t* lds = (const uint32_t*)smem;
    const uint32_t boff = q * rb + blk * fmt_block_bytes(F);
    uint64_t best = 0;
    for (uint32_t st = 0; st < nsteps; st++) {
        wait_vm(2u * (kHeadSlots - 1));   // step st (the oldest in flight) has landed
        const uint32_t so = soff + (st % kHeadSlots) * kSlotBytes;
        float a[1] = {0.f};
        unit_dot<1>(F, lds, so + boff, j, lds, xr, sx, a);
        const float v = reduce_scatter_k<1, KU>(a);
        const uint32_t row = (gw + st * nwv) * rps + q;
        if (unit == 0 && row < rows) {
            logits[row] = v;
            best = max_u64(best, amax_key(v, row));
        }
        stage_group(smem + so, src(st + kHeadSlots), gbytes);   // after this slot's reads
    }
    wait_vm(0);
    best = wave_max_u64(best);
    if (lane == 0) part[gw] = best;
}

// ---- output head, Q6_K rows of 2048 columns: bf16 MFMA -------------------------
// A 16-row tile and one 256-column block (a "unit") at a time, per wave.
// For each 32-column run r of the block (qw6's even-scale rule gives a run one
// scale), one v_mfma_f32_16x16x32_bf16 with
//   B[k][n] = 128 + q (bf16, exact) of row n, column 32 r + k of the block,
//   A[c][k] = part c / 8 (hi, lo) of the normalised activation of column
//             32 (c % 8) + k of the block,
// so that D_r[c][n] for c % 8 == r is row n's product with run r, part c / 8
// (the other entries are not used). A is the same for every tile: eight 4-VGPR
// operands per lane, built once. A ninth MFMA with B = -160 (the code bias 128
// plus Q6_K's 32) gives -160 x each A row's sum, and seeds every D_r with it.
// The run's d * scale multiplies its entry afterwards; the four lane groups
// (hi / lo, runs 0-3 / 4-7) add up a row at the end (qw6_vk.c:3447-3478 is the
// reference's head; the arithmetic is qw6.c:1550-1578 and 2490-2492).
// Units stream through kHqSlots direct-to-LDS slots per wave: 16 rows x 15
// chunks of 16 B (the block spans 14; the 15th, a repeat of the row's first,
// spaces the rows over the LDS banks).
constexpr uint32_t kHqChunks = 15;
constexpr uint32_t kHqSlot = 4096;          // bytes per slot (240 chunks, padded)
constexpr uint32_t kHqSlots = 4;            // units in flight per wave
constexpr uint32_t kHqWG = 4;               // waves per workgroup
constexpr uint32_t kHqLoads = 4;            // 16-B loads per lane per unit
constexpr uint32_t kHqWaves = 2048;         // waves of one launch, at most
constexpr uint32_t kHqRowBytes = 8 * 210;   // a Q6_K row of 2048 columns

// Stage block b of tile `tile` (16 rows from W + 16 tile rows) into slot.
// The block starts 2b bytes into its first 16-B chunk (W 16-byte aligned).
__device__ __forceinline__ void hq_stage(uint8_t* slot, const uint8_t* W, uint32_t tile, uint32_t b) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint8_t* c0 = W + (size_t)tile * 16u * kHqRowBytes + 208u * b;   // 16-aligned: 210 b - 2 b
#pragma unroll
    for (uint32_t k = 0; k < kHqLoads; k++) {
        const uint32_t i = 64u * k + lane;   // chunk i: row i / 15, chunk i % 15
        const uint32_t row = i < 16u * kHqChunks ? i / kHqChunks : 0u;
        const uint32_t ch = i % kHqChunks < 14u ? i % kHqChunks : 0u;
        __builtin_amdgcn_global_load_lds((glb_void_t*)(c0 + (size_t)row * kHqRowBytes + 16u * ch),
                                         (lds_void_t*)(slot + 1024u * k), 16, 0, 0);
    }
}

// Two dwords from 8 bytes at LDS byte offset o, o % 4 == 2 * (B & 1).
template <uint32_t B>
__device__ __forceinline__ uint2 hq_read8(const uint32_t* s, uint32_t o) {
    if constexpr ((B & 1u) == 0) {
        return make_uint2(s[o >> 2], s[(o >> 2) + 1]);
    } else {
        const uint32_t i = o >> 2, w0 = s[i], w1 = s[i + 1], w2 = s[i + 2];
        return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, 2), __builtin_amdgcn_alignbyte(w2, w1, 2));
    }
}

// The bytes of block B of a unit this lane needs (row n at LDS byte offset
// o_row): ql of runs 4h + 0 / 2 (a) and 4h + 1 / 3 (c), qh (h), for halves h;
// scales 8 hs + 0, 2, 4, 6 (hs = g & 1, the runs of its D entries); d.
struct HqRaw {
    uint2 a[2], c[2], h[2], sc;
    uint32_t dw;
};
template <uint32_t B>
__device__ __forceinline__ HqRaw hq_load(const uint32_t* s, uint32_t o_row, uint32_t g) {
    const uint32_t o = o_row + 2u * B;   // the block's first byte
    HqRaw r;
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        r.a[h] = hq_read8<B>(s, o + 64u * h + 8u * g);
        r.c[h] = hq_read8<B>(s, o + 64u * h + 32u + 8u * g);
        r.h[h] = hq_read8<B>(s, o + 128u + 32u * h + 8u * g);
    }
    r.sc = hq_read8<B>(s, o + 192u + 8u * (g & 1u));
    r.dw = s[(o + 208u) >> 2];
    return r;
}

// Block B's products from its bytes: adds this lane's share of row n's dot
// product with the block to acc.
template <uint32_t B>
__device__ __forceinline__ void hq_math(const HqRaw& r, uint32_t g, const uint4& a, float& acc) {
    const uint4 bias = u4(0xC320C320u, 0xC320C320u, 0xC320C320u, 0xC320C320u);   // bf16 -160
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    const f32x4 db = mfma(a, bias, z4);
    f32x4 D[8];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        // runs 4h .. 4h + 3: low / high nibbles of a (runs 0, 2) and c (1, 3),
        // two bits of qh per run (qw6.c:1550-1578)
        const uint32_t av[2] = {r.a[h].x, r.a[h].y}, cv[2] = {r.c[h].x, r.c[h].y};
        const uint32_t hv[2] = {r.h[h].x, r.h[h].y};
        uint32_t w[4][2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            w[0][i] = (av[i] & 0x0f0f0f0fu) | ((hv[i] & 0x03030303u) << 4);
            w[1][i] = (cv[i] & 0x0f0f0f0fu) | ((hv[i] & 0x0c0c0c0cu) << 2);
            w[2][i] = ((av[i] >> 4) & 0x0f0f0f0fu) | (hv[i] & 0x30303030u);
            w[3][i] = ((cv[i] >> 4) & 0x0f0f0f0fu) | ((hv[i] >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) D[4 * h + k] = mfma(a, codes8(w[k][0], w[k][1]), db);
    }
    // lane (n, g) holds D[4g + v][n]: part g / 2 of run 4 (g & 1) + v
    const uint32_t hs = g & 1u;
    const float d = h2f((r.dw >> (16u * (B & 1u))) & 0xffffu);   // byte 208 + 2B of a 4-aligned row
    float t = 0.f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const float val = hs ? D[4 + v][v] : D[v][v];
        const uint32_t wv = v < 2 ? r.sc.x : r.sc.y;
        const float sc = (float)(int8_t)((wv >> (16 * (v & 1))) & 0xffu);
        t = fmaf(sc, val, t);
    }
    acc = fmaf(d, t, acc);
}

// LDS reads of this wave done (before a slot they read is restaged).
__device__ __forceinline__ void wait_lgkm0() {
    __builtin_amdgcn_s_waitcnt(0xc07fu);   // lgkmcnt(0); vmcnt, expcnt not waited
    asm volatile("" ::: "memory");
}

// Unit u = 8 st + B (block B of this step's tile) with its bytes in r:
// restage its slot with unit u + S, read unit u + 1's bytes (landed once at
// most S - 1 units remain in flight) into rn, then multiply block B.
template <uint32_t S, uint32_t B>
__device__ __forceinline__ void hq_step(const uint32_t* s, uint8_t* slots, uint32_t so, uint32_t g,
                                        const uint4 (&A)[8], float& acc, HqRaw& r, const uint8_t* W,
                                        uint32_t tile_next, uint32_t tile_now, uint32_t tiles) {
    wait_lgkm0();
    const uint32_t t = B + S < 8 ? tile_now : tile_next;
    hq_stage(slots + (B % S) * kHqSlot, W, t < tiles ? t : 0u, (B + S) % 8);
    wait_vm((S - 1) * kHqLoads);
    const HqRaw rn = hq_load<(B + 1) % 8>(s, so + ((B + 1) % S) * kHqSlot, g);
    hq_math<B>(r, g, A[B], acc);
    r = rn;
}

// S: units in flight per wave (4 or 8), NW: waves per workgroup; built for
// two waves per SIMD (at most 256 registers).
template <uint32_t S, uint32_t NW>
__global__ __launch_bounds__(64 * NW, 2) void k_head_q6k(const uint8_t* __restrict__ W, uint32_t tiles,
                                                      uint32_t nsteps, const float* __restrict__ x,
                                                      const float* __restrict__ norm_w, float eps,
                                                      float* __restrict__ logits,
                                                      uint64_t* __restrict__ part) {
    static_assert(S == 4 || S == 8, "a slot per block or per half of the blocks");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4, c = lane & 15u;
    const uint32_t gw = blockIdx.x * NW + wave, nwv = gridDim.x * NW;
    uint8_t* slots = smem + wave * S * kHqSlot;
    const uint32_t so = (uint32_t)(slots - smem) + 240u * n;   // row n in slot 0
    auto tile_of = [&](uint32_t st) { return gw + st * nwv; };
    // the first S units of step 0 in flight first
#pragma unroll
    for (uint32_t b = 0; b < S; b++) {
        const uint32_t t = tile_of(0);
        hq_stage(slots + b * kHqSlot, W, t < tiles ? t : 0u, b);
    }
    // A operands: lane (c, g) holds part c / 8 of columns 256 b + 32 (c % 8) + 8 g .. + 8
    float xv[8][8];
    float ss = 0.f;
#pragma unroll
    for (uint32_t b = 0; b < 8; b++) {
        const float* xp = x + 256u * b + 32u * (c & 7u) + 8u * g;
        const float4 u0 = *(const float4*)xp, u1 = *(const float4*)(xp + 4);
        xv[b][0] = u0.x; xv[b][1] = u0.y; xv[b][2] = u0.z; xv[b][3] = u0.w;
        xv[b][4] = u1.x; xv[b][5] = u1.y; xv[b][6] = u1.z; xv[b][7] = u1.w;
#pragma unroll
        for (int j = 0; j < 8; j++) ss = fmaf(xv[b][j], xv[b][j], ss);
    }
    if (norm_w) {   // final RMSNorm (qw6.c:2490-2492); every column appears in two lanes
        ss = group_sum<64>(ss) * 0.5f;
        const float sc = 1.0f / sqrtf(ss / 2048.0f + eps);
#pragma unroll
        for (uint32_t b = 0; b < 8; b++) {
            const float* wp = norm_w + 256u * b + 32u * (c & 7u) + 8u * g;
            const float4 u0 = *(const float4*)wp, u1 = *(const float4*)(wp + 4);
            const float wv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) xv[b][j] = xv[b][j] * sc * wv[j];
        }
    }
    uint4 A[8];
    const bool lo = c >= 8;
#pragma unroll
    for (uint32_t b = 0; b < 8; b++) {
        uint32_t wd[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float x0 = xv[b][2 * i], x1 = xv[b][2 * i + 1];
            const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
            const __bf16 l0 = (__bf16)(x0 - (float)h0), l1 = (__bf16)(x1 - (float)h1);
            wd[i] = lo ? (bfb(l0) | (bfb(l1) << 16)) : (bfb(h0) | (bfb(h1) << 16));
        }
        A[b] = u4(wd[0], wd[1], wd[2], wd[3]);
    }
    const uint32_t* s = (const uint32_t*)smem;
    wait_vm((S - 1) * kHqLoads);   // unit 0 has landed
    HqRaw r = hq_load<0>(s, so, g);
    uint64_t best = 0;
    for (uint32_t st = 0; st < nsteps; st++) {
        const uint32_t tn = tile_of(st), tx = tile_of(st + 1);
        float acc = 0.f;
        hq_step<S, 0>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 1>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 2>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 3>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 4>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 5>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 6>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        hq_step<S, 7>(s, slots, so, g, A, acc, r, W, tx, tn, tiles);
        acc += partner(acc, 16, lane);
        acc += partner(acc, 32, lane);
        if (g == 0 && tn < tiles) {
            const uint32_t row = 16u * tn + n;
            logits[row] = acc;
            best = max_u64(best, amax_key(acc, row));
        }
    }
    wait_vm(0);   // no LDS-direct load lands after the workgroup ends
    best = wave_max_u64(best);
    if (lane == 0) part[gw] = best;
}

__global__ void k_gather(const float* eo, const float* ew, const float* sh, float sw,
                         float* o, uint32_t dim, uint32_t top_k) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    float acc = 0.f;
    for (uint32_t e = 0; e < top_k; e++) acc = fmaf(ew[e], eo[(size_t)e * dim + i], acc);
    if (sh) acc = fmaf(sw, sh[i], acc);
    o[i] = acc;
}

__global__ __launch_bounds__(kWG) void k_rmsnorm(const float* x, const float* w, float* y,
                                                 uint32_t n, float eps) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += kWG) ss = fmaf(xr[i], xr[i], ss);
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float sc = 1.0f / sqrtf(tot / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += kWG) yr[i] = xr[i] * sc * w[i];
}

// ---- synthetic data --------------------------------------------------------------

__global__ void k_synth_blocks(uint8_t* dst, int fmt, uint64_t nblocks, uint64_t first,
                               uint64_t key, uint32_t bb) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint64_t gb = first + b;
    uint8_t* o = dst + b * bb;
    for (uint32_t w = 0; w * 8 < bb; w++) {
        const uint64_t h = sm_hash(key, gb * 40 + w);
        for (uint32_t k = 0; k < 8 && w * 8 + k < bb; k++) o[w * 8 + k] = (uint8_t)(h >> (8 * k));
    }
    struct Field { uint32_t off; float scale; };
    Field fl[2];
    int nf;
    switch (fmt) {
    case F_Q4K: case F_Q5K: fl[0] = {0, 2e-3f}; fl[1] = {2, 2e-3f}; nf = 2; break;
    case F_Q6K: fl[0] = {208, 1e-3f}; nf = 1; break;
    case F_IQ2XXS: fl[0] = {0, 2e-3f}; nf = 1; break;
    default: fl[0] = {0, 1e-3f}; nf = 1; break;
    }
    for (int f = 0; f < nf; f++) {
        const float z = sm_normal(key, gb * 40 + 28 + 3 * f);
        const uint16_t h = f2h_rne(fabsf(z) * fl[f].scale);
        o[fl[f].off] = (uint8_t)h;
        o[fl[f].off + 1] = (uint8_t)(h >> 8);
    }
}

__global__ void k_synth_normal(float* dst, uint64_t n, float mean, float sd, uint64_t key) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    {   // two roundings, as the host generator (no fused multiply-add)
#pragma clang fp contract(off)
        const float z = sm_normal(key, 3 * i) * sd;
        dst[i] = mean == 0.f ? z : mean + z;
    }
}

}  // namespace

int qw6::qw6_fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const int r = vfail(fmt, ap);
    va_end(ap);
    return r;
}

// ==================================================================================
// Host side
// ==================================================================================

struct qw6_hip_ctx_s {
    int device;
    uint32_t max_tokens;
    int mode;
    std::vector<void*> owned;
    // decode workspace
    float* logits;
    float* sw;
    float* xn;
    SlotTable* slots;
    float* mid;
    uint32_t ws_hidden, ws_inter;
    // small-batch MFMA operands (k_mx_*)
    uint4* mxa;
    uint16_t* mxs;
    uint4* mma;
    uint16_t* mms;
    uint32_t mx_hidden, mx_inter;
    // batched (grouped MFMA) workspace, sized for max_tokens
    PrefillWs pre;
    uint32_t pre_hidden, pre_inter, pre_experts;
    // per-kernel timing (qw6_hip_profile)
    std::vector<hipEvent_t> prof_ev;
    uint32_t prof_cap, prof_calls;
    // argmax partial maxima; output head's normalised input
    uint64_t* amax_part;
    float* head_x;
    uint32_t head_hidden;
    // this device's copy of the static decode workspace (qw6_hip_moe_forward_noalloc)
    uint8_t* scratch;
};

int qw6::ctx_device(const qw6_hip_ctx_t* c) { return c->device; }

struct qw6_hip_experts_s {
    qw6_hip_ctx_t* ctx;
    ExpertEnt* dev;
    uint32_t n;
    uint32_t hidden, inter;
    uint32_t tmask_gu, tmask_dn;
    uint32_t rb_gu_max;   // widest gate/up row in bytes
    uint32_t rb_dn_max;   // widest down row in bytes
    int fmt_gu, fmt_dn;   // the single gate/up (down) format, -1 if mixed
    uint32_t fmask_gu, fmask_dn;   // the formats present: bit f (bit 31: one the grouped path lacks)
    int xl_dn;            // a down format whose activation layout every expert's
                          // down format shares (the IQ formats share one), or -1
    int gu_same;          // every expert's gate and up share a format
    PackRef pk[3];        // regular-pack addressing per matrix kind
};

namespace {

struct DevGuard {
    int prev = -1;
    explicit DevGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DevGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

int check_matrix(int quant, uint32_t rows, uint32_t cols, int* fmt) {
    if (rows == 0 || cols == 0) return fail("empty matrix (%u x %u)", rows, cols);
    if (cols % 256) return fail("cols %% 256 != 0 (cols = %u)", cols);
    const int f = fmt_of_quant(quant);
    if (f < 0 && quant != 0) return fail("unsupported quant %d", quant);
    *fmt = f;
    return 0;
}

bool fast_k(uint32_t K) { return K == 256 || K == 512 || K == 1024 || K == 2048; }

template <int V> using IC = std::integral_constant<int, V>;

// Run fn(IC<T>, IC<F>) for the kernel instantiation of T tokens and format
// f: format-specialised kernels for 1-2 tokens, the format switch otherwise
// (or when f < 0: mixed formats).
template <typename Fn>
void launch_by_fmt(int f, uint32_t T, Fn fn) {
    if (T <= 2 && f >= 0) {
        auto by_f = [&](auto tc) {
            switch (f) {
            case F_Q4K: fn(tc, IC<F_Q4K>{}); break;
            case F_Q5K: fn(tc, IC<F_Q5K>{}); break;
            case F_Q6K: fn(tc, IC<F_Q6K>{}); break;
            case F_IQ2XXS: fn(tc, IC<F_IQ2XXS>{}); break;
            case F_IQ2S: fn(tc, IC<F_IQ2S>{}); break;
            default: fn(tc, IC<F_IQ3S>{}); break;
            }
        };
        if (T == 1) by_f(IC<1>{});
        else by_f(IC<2>{});
        return;
    }
    switch (T) {
    case 1: fn(IC<1>{}, IC<-1>{}); break;
    case 2: fn(IC<2>{}, IC<-1>{}); break;
    case 3: fn(IC<3>{}, IC<-1>{}); break;
    default: fn(IC<4>{}, IC<-1>{}); break;
    }
}

// Launch y = W x for n_tok tokens on device data (W.fmt < 0: F32).
int launch_matvec(const MatD& W, const float* x, float* y, uint32_t n_tok, hipStream_t st) {
    for (uint32_t t0 = 0; t0 < n_tok; t0 += kMaxTok) {
        const uint32_t T = n_tok - t0 < kMaxTok ? n_tok - t0 : kMaxTok;
        const float* xt = x + (size_t)t0 * W.cols;
        float* yt = y + (size_t)t0 * W.rows;
        // per-chunk y layout: [t][rows] with t relative to chunk
        if (W.fmt < 0) {
            const float* wf = (const float*)W.p;
            switch (T) {
            case 1: k_matvec_f32<1><<<W.rows, 64, 0, st>>>(wf, xt, yt, W.rows, W.cols); break;
            case 2: k_matvec_f32<2><<<W.rows, 64, 0, st>>>(wf, xt, yt, W.rows, W.cols); break;
            case 3: k_matvec_f32<3><<<W.rows, 64, 0, st>>>(wf, xt, yt, W.rows, W.cols); break;
            default: k_matvec_f32<4><<<W.rows, 64, 0, st>>>(wf, xt, yt, W.rows, W.cols); break;
            }
        } else {
            const uint32_t tmask = fmt_table_mask(W.fmt);
            const uint32_t toff = tab_bytes(tmask);
            if (fast_k(W.cols)) {
                const uint32_t U = W.cols / 32, rps = 64 / U;
                const uint32_t R = 4 * rps * kStepsMv;   // multiple of 16 bytes: 32*steps*bb
                const size_t lds = toff + align16(R * W.rb) + 16 + T * W.cols * 4 + 16;
                if (lds > kLdsBudget) return fail("matvec tile exceeds LDS budget");
                const dim3 grid((W.rows + R - 1) / R);
                launch_by_fmt(W.fmt, T, [&](auto tc, auto fc) {
                    k_matvec<decltype(tc)::value, decltype(fc)::value>
                        <<<grid, kWG, lds, st>>>(W, xt, yt, R, tmask);
                });
            } else {
                const size_t lds = toff + W.rb + 32;
                if (lds > kLdsBudget) return fail("row too large for the generic kernel (%u B)", W.rb);
                switch (T) {
                case 1: k_matvec_generic<1><<<W.rows, 64, lds, st>>>(W, xt, yt, tmask); break;
                case 2: k_matvec_generic<2><<<W.rows, 64, lds, st>>>(W, xt, yt, tmask); break;
                case 3: k_matvec_generic<3><<<W.rows, 64, lds, st>>>(W, xt, yt, tmask); break;
                default: k_matvec_generic<4><<<W.rows, 64, lds, st>>>(W, xt, yt, tmask); break;
                }
            }
        }
        CK(hipGetLastError());
    }
    return 0;
}

// Two passes over n >= 1 floats: at most kArgmaxBlocks partial maxima, then one
// block over them. part: kArgmaxBlocks words of scratch.
int launch_argmax(const float* x, uint32_t n, uint64_t* part, uint32_t* out, hipStream_t st) {
    const uint32_t nb = std::min(kArgmaxBlocks, (n + 1023u) / 1024u);
    k_argmax_part<<<nb, 256, 0, st>>>(x, n, part);
    k_argmax_final<<<1, 256, 0, st>>>(x, part, nb, out);
    CK(hipGetLastError());
    return 0;
}

// The output head's streaming pass (k_head) and the argmax of its per-wave
// keys. Needs a GGUF format, cols in {256, 512, 1024, 2048} and rows a
// multiple of the rows per step; returns 1 when the shape does not fit.
// part: kHeadWaves words.
int launch_head(const MatD& W, const float* x, const float* norm_w, float eps, float* logits,
                uint64_t* part, uint32_t* out, hipStream_t st) {
    if (W.fmt == F_Q6K && W.cols == 2048 && W.rows % 16 == 0 && ((uintptr_t)W.p & 15u) == 0 &&
        ((uintptr_t)x & 15u) == 0 && ((uintptr_t)norm_w & 15u) == 0) {
        // bf16-MFMA head: 16-row tiles, each wave a tile per step
        const uint32_t tiles = W.rows / 16;
        const uint32_t nwv = std::min(kHqWaves, (tiles + kHqWG - 1) / kHqWG * kHqWG);
        const uint32_t nsteps = (tiles + nwv - 1) / nwv;
        k_head_q6k<kHqSlots, kHqWG><<<nwv / kHqWG, 64 * kHqWG, kHqWG * kHqSlots * kHqSlot, st>>>(
            W.p, tiles, nsteps, x, norm_w, eps, logits, part);
        k_argmax_final<<<1, 256, 0, st>>>(logits, part, nwv, out);
        CK(hipGetLastError());
        return 0;
    }
    if (W.fmt < 0 || !fast_k(W.cols)) return 1;
    const uint32_t U = W.cols / 32, rps = 64 / U;
    if (W.rows % rps) return 1;
    const uint32_t groups = W.rows / rps;
    const uint32_t nwv = std::min(kHeadWaves, std::max(4u, (groups + 7) / 8 / 4 * 4));
    const uint32_t nsteps = (groups + nwv - 1) / nwv;
    const uint32_t tmask = fmt_table_mask(W.fmt);
    const size_t lds = tab_bytes(tmask) + 4 * kHeadSlots * kSlotBytes;
    auto go = [&](auto fc, auto kc) {
        k_head<decltype(fc)::value, decltype(kc)::value><<<nwv / 4, kWG, lds, st>>>(
            W.p, groups, W.rows, W.rb, nsteps, x, norm_w, eps, logits, part, tmask);
    };
    auto by_k = [&](auto fc) {
        switch (U) {
        case 8: go(fc, IC<8>{}); break;
        case 16: go(fc, IC<16>{}); break;
        case 32: go(fc, IC<32>{}); break;
        default: go(fc, IC<64>{}); break;
        }
    };
    switch (W.fmt) {
    case F_Q4K: by_k(IC<F_Q4K>{}); break;
    case F_Q5K: by_k(IC<F_Q5K>{}); break;
    case F_Q6K: by_k(IC<F_Q6K>{}); break;
    case F_IQ2XXS: by_k(IC<F_IQ2XXS>{}); break;
    case F_IQ2S: by_k(IC<F_IQ2S>{}); break;
    default: by_k(IC<F_IQ3S>{}); break;
    }
    k_argmax_final<<<1, 256, 0, st>>>(logits, part, nwv, out);
    CK(hipGetLastError());
    return 0;
}

struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

int host_matvec(int quant, const void* w, const float* x, float* y, uint32_t rows,
                uint32_t cols) {
    if (!w || !x || !y) return fail("null pointer");
    int f;
    if (check_matrix(quant, rows, cols, &f)) return -1;
    const size_t rb = quant == 0 ? (size_t)cols * 4 : (size_t)(cols / 256) * fmt_block_bytes(f);
    DevBuf bw, bx, by;
    CK(hipMalloc(&bw.p, rows * rb + 16));
    CK(hipMalloc(&bx.p, (size_t)cols * 4));
    CK(hipMalloc(&by.p, (size_t)rows * 4));
    CK(hipMemcpy(bw.p, w, rows * rb, hipMemcpyHostToDevice));
    CK(hipMemcpy(bx.p, x, (size_t)cols * 4, hipMemcpyHostToDevice));
    const MatD W = {(const uint8_t*)bw.p, quant == 0 ? -1 : f, rows, cols, (uint32_t)rb};
    if (launch_matvec(W, (const float*)bx.p, (float*)by.p, 1, nullptr)) return -1;
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(y, by.p, (size_t)rows * 4, hipMemcpyDeviceToHost));
    return 0;
}

int alloc_owned(qw6_hip_ctx_t* c, size_t bytes, void** p) {
    CK(hipMalloc(p, bytes ? bytes : 16));
    c->owned.push_back(*p);
    CK(hipMemset(*p, 0, bytes ? bytes : 16));
    return 0;
}

// ---- the static decode workspace -------------------------------------------------
// qw6_hip_moe_forward_noalloc runs the per-token kernels on a workspace that
// is a file-scope device array instead of context allocations. Every device
// the library runs on holds its own copy of the array (at its own address)
// until the process ends. Host code never uses the array's name as an
// address: each device's address comes from hipGetSymbolAddress, taken once
// per device with that device current (at qw6_hip_ctx_init).
constexpr size_t kScratchBytes = (size_t)4 << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
uint8_t* g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// The address of `scratch` on `device` (which must be current).
int scratch_address(int device, uint8_t** out) {
    if (device < 0 || device >= kMaxDevices) return fail("device %d beyond the static workspace table", device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[device]) {
        void* p = nullptr;
        CK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail("no device address for the static workspace");
        g_scratch_addr[device] = (uint8_t*)p;
    }
    *out = g_scratch_addr[device];
    return 0;
}

// Per-token decode workspace carved from one region (256-byte aligned
// pieces): the same buffers ensure_ws and ensure_mx_ws allocate one by one.
struct DecodeWs {
    float* logits;
    float* sw;
    float* xn;
    SlotTable* slots;
    float* mid;
    uint4* mxa;
    uint16_t* mxs;
    uint4* mma;
    uint16_t* mms;
};

size_t carve_decode_ws(uint8_t* base, uint32_t hidden, uint32_t inter, DecodeWs* w) {
    size_t o = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = base ? base + o : nullptr;
        o += (bytes + 255) & ~(size_t)255;
        return p;
    };
    DecodeWs d;
    d.logits = (float*)take((size_t)kSplitMaxTok * 256 * 4);
    d.sw = (float*)take(kSplitMaxTok * 4);
    d.xn = (float*)take((size_t)kSplitMaxTok * hidden * 4);
    d.slots = (SlotTable*)take(kSplitMaxTok * sizeof(SlotTable));   // one per token (fp32 kernels)
    d.mid = (float*)take((size_t)kMidRows * inter * 4);
    d.mxa = (uint4*)take((size_t)(hidden / 32) * 64 * 16);
    d.mxs = (uint16_t*)take((size_t)(hidden / 256) * 192 * 2);
    d.mma = (uint4*)take((size_t)(kMaxSlots + 1) * (inter / 32) * 64 * 16);
    d.mms = (uint16_t*)take((size_t)(kMaxSlots + 1) * (inter / 256) * 192 * 2);
    if (w) *w = d;
    return o;
}

int ensure_argmax_ws(qw6_hip_ctx_t* c) {
    if (c->amax_part) return 0;
    void* p;
    if (alloc_owned(c, (size_t)std::max(kArgmaxBlocks, kHeadWaves) * 8, &p)) return -1;
    c->amax_part = (uint64_t*)p;
    return 0;
}

}  // namespace

extern "C" {

const char* qw6_hip_last_error(void) { return g_err; }

#ifdef QW6_TRACE
int qw6_hip_trace_read(void* host) {
    CK(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), sizeof(g_trace)));
    return 0;
}
int qw6_hip_mark_read(void* host) {
    CK(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_mark), sizeof(g_mark)));
    return 0;
}
int qw6_hip_trace_clear(void) {
    static unsigned long long z[4][4096][2];
    CK(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), z, sizeof(z)));
    return 0;
}
#endif

int qw6_hip_matvec_f32_host(const float* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols) {
    if (!w || !x || !y) return fail("null pointer");
    if (rows == 0 || cols == 0) return fail("empty matrix");
    DevBuf bw, bx, by;
    CK(hipMalloc(&bw.p, (size_t)rows * cols * 4));
    CK(hipMalloc(&bx.p, (size_t)cols * 4));
    CK(hipMalloc(&by.p, (size_t)rows * 4));
    CK(hipMemcpy(bw.p, w, (size_t)rows * cols * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(bx.p, x, (size_t)cols * 4, hipMemcpyHostToDevice));
    const MatD W = {(const uint8_t*)bw.p, -1, rows, cols, cols * 4};
    if (launch_matvec(W, (const float*)bx.p, (float*)by.p, 1, nullptr)) return -1;
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(y, by.p, (size_t)rows * 4, hipMemcpyDeviceToHost));
    return 0;
}

int qw6_hip_matmul_q4k_host(const void* w, const float* x, float* y, uint32_t r, uint32_t c) {
    return host_matvec(4, w, x, y, r, c);
}
int qw6_hip_matmul_q5k_host(const void* w, const float* x, float* y, uint32_t r, uint32_t c) {
    return host_matvec(6, w, x, y, r, c);
}
int qw6_hip_matmul_q6k_host(const void* w, const float* x, float* y, uint32_t r, uint32_t c) {
    return host_matvec(7, w, x, y, r, c);
}
int qw6_hip_matmul_iq2xxs_host(const void* w, const float* x, float* y, uint32_t r, uint32_t c) {
    return host_matvec(13, w, x, y, r, c);
}
int qw6_hip_matmul_iq2s_host(const void* w, const float* x, float* y, uint32_t r, uint32_t c) {
    return host_matvec(11, w, x, y, r, c);
}
int qw6_hip_matmul_iq3s_host(const void* w, const float* x, float* y, uint32_t r, uint32_t c) {
    return host_matvec(9, w, x, y, r, c);
}

int qw6_hip_silu_mul_host(const float* gate, const float* up, float* out, uint32_t n) {
    if (!gate || !up || !out) return fail("null pointer");
    if (n == 0) return fail("n == 0");
    DevBuf bg, bu, bo;
    CK(hipMalloc(&bg.p, (size_t)n * 4));
    CK(hipMalloc(&bu.p, (size_t)n * 4));
    CK(hipMalloc(&bo.p, (size_t)n * 4));
    CK(hipMemcpy(bg.p, gate, (size_t)n * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(bu.p, up, (size_t)n * 4, hipMemcpyHostToDevice));
    k_silu_mul<<<(n + 255) / 256, 256>>>((const float*)bg.p, (const float*)bu.p, (float*)bo.p, n);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(out, bo.p, (size_t)n * 4, hipMemcpyDeviceToHost));
    return 0;
}

int qw6_hip_moe_route_host(const float* logits, uint32_t* indices, float* weights,
                           uint32_t n_experts, uint32_t top_k) {
    if (!logits || !indices || !weights) return fail("null pointer");
    if (n_experts == 0 || n_experts > 256 || top_k == 0 || top_k > n_experts || top_k > 8)
        return fail("moe_route bounds (n_experts %u, top_k %u)", n_experts, top_k);
    DevBuf bl, bi, bw;
    CK(hipMalloc(&bl.p, (size_t)n_experts * 4));
    CK(hipMalloc(&bi.p, (size_t)top_k * 4));
    CK(hipMalloc(&bw.p, (size_t)top_k * 4));
    CK(hipMemcpy(bl.p, logits, (size_t)n_experts * 4, hipMemcpyHostToDevice));
    k_route<<<1, 64>>>((const float*)bl.p, n_experts, top_k, (uint32_t*)bi.p, (float*)bw.p);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(indices, bi.p, (size_t)top_k * 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(weights, bw.p, (size_t)top_k * 4, hipMemcpyDeviceToHost));
    return 0;
}

int qw6_hip_moe_gather_host(const float* expert_out, const float* expert_weights,
                            const float* shared_out, float shared_weight, float* out,
                            uint32_t dim, uint32_t top_k) {
    if (!expert_out || !expert_weights || !out) return fail("null pointer");
    if (dim == 0 || top_k == 0 || top_k > 8) return fail("moe_gather bounds");
    DevBuf be, bw, bs, bo;
    CK(hipMalloc(&be.p, (size_t)top_k * dim * 4));
    CK(hipMalloc(&bw.p, (size_t)top_k * 4));
    CK(hipMalloc(&bo.p, (size_t)dim * 4));
    CK(hipMemcpy(be.p, expert_out, (size_t)top_k * dim * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(bw.p, expert_weights, (size_t)top_k * 4, hipMemcpyHostToDevice));
    if (shared_out) {
        CK(hipMalloc(&bs.p, (size_t)dim * 4));
        CK(hipMemcpy(bs.p, shared_out, (size_t)dim * 4, hipMemcpyHostToDevice));
    }
    k_gather<<<(dim + 255) / 256, 256>>>((const float*)be.p, (const float*)bw.p,
                                         (const float*)bs.p, shared_weight, (float*)bo.p, dim,
                                         top_k);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(out, bo.p, (size_t)dim * 4, hipMemcpyDeviceToHost));
    return 0;
}

int qw6_hip_rmsnorm_host(const float* x, const float* w, float* y, uint32_t n, float eps) {
    if (!x || !w || !y) return fail("null pointer");
    if (n == 0) return fail("n == 0");
    DevBuf bx, bw, by;
    CK(hipMalloc(&bx.p, (size_t)n * 4));
    CK(hipMalloc(&bw.p, (size_t)n * 4));
    CK(hipMalloc(&by.p, (size_t)n * 4));
    CK(hipMemcpy(bx.p, x, (size_t)n * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(bw.p, w, (size_t)n * 4, hipMemcpyHostToDevice));
    k_rmsnorm<<<1, kWG>>>((const float*)bx.p, (const float*)bw.p, (float*)by.p, n, eps);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(y, by.p, (size_t)n * 4, hipMemcpyDeviceToHost));
    return 0;
}

// ---- context -------------------------------------------------------------------

int qw6_hip_ctx_init(qw6_hip_ctx_t** out, int device, uint32_t max_tokens) {
    if (!out) return fail("null ctx pointer");
    *out = nullptr;
    int n = 0;
    CK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail("device %d not present (%d devices)", device, n);
    if (max_tokens == 0) return fail("max_tokens == 0");
    DevGuard g(device);
    uint8_t* sp = nullptr;
    if (scratch_address(device, &sp)) return -1;
    qw6_hip_ctx_t* c = new qw6_hip_ctx_t();
    c->device = device;
    c->max_tokens = max_tokens;
    c->mode = 0;
    c->scratch = sp;
    *out = c;
    return 0;
}

void qw6_hip_ctx_free(qw6_hip_ctx_t* c) {
    if (!c) return;
    DevGuard g(c->device);
    for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
    for (void* p : c->owned) (void)hipFree(p);
    delete c;
}

int qw6_hip_upload(qw6_hip_ctx_t* c, const void* host, size_t bytes, void** dev) {
    if (!c || !host || !dev) return fail("null pointer");
    DevGuard g(c->device);
    if (alloc_owned(c, bytes, dev)) return -1;
    CK(hipMemcpy(*dev, host, bytes, hipMemcpyHostToDevice));
    return 0;
}

int qw6_hip_alloc(qw6_hip_ctx_t* c, size_t bytes, void** dev) {
    if (!c || !dev) return fail("null pointer");
    DevGuard g(c->device);
    return alloc_owned(c, bytes, dev);
}

int qw6_hip_set_mode(qw6_hip_ctx_t* c, int mode) {
    if (!c || mode < 0 || mode > 3) return fail("bad mode");
    c->mode = mode;
    return 0;
}

int qw6_hip_matvec(qw6_hip_ctx_t* c, const qw6_hip_matrix_t* w, const float* x, float* y,
                   uint32_t n_tok, void* stream) {
    if (!c || !w || !w->data || !x || !y) return fail("null pointer");
    if (n_tok == 0) return 0;
    int f;
    if (check_matrix(w->quant, w->rows, w->cols, &f)) return -1;
    if ((uintptr_t)w->data & 15u) return fail("weight data not 16-byte aligned");
    // the quantized kernels read the activations in 16-byte pieces
    if (w->quant != 0 && ((uintptr_t)x & 15u)) return fail("x must be 16-byte aligned");
    DevGuard g(c->device);
    const uint32_t rb = w->quant == 0 ? w->cols * 4 : (w->cols / 256) * fmt_block_bytes(f);
    const MatD W = {(const uint8_t*)w->data, w->quant == 0 ? -1 : f, w->rows, w->cols, rb};
    return launch_matvec(W, x, y, n_tok, (hipStream_t)stream);
}

int qw6_hip_experts_create(qw6_hip_ctx_t* c, const qw6_hip_matrix_t* gate,
                           const qw6_hip_matrix_t* up, const qw6_hip_matrix_t* down,
                           uint32_t n_experts, qw6_hip_experts_t** out) {
    if (!c || !gate || !up || !down || !out) return fail("null pointer");
    *out = nullptr;
    if (n_experts == 0 || n_experts > 256) return fail("n_experts %u not in 1..256", n_experts);
    const uint32_t hidden = gate[0].cols, inter = gate[0].rows;
    std::vector<ExpertEnt> tab(n_experts);
    uint32_t mgu = 0, mdn = 0, rb_gu = 0, rb_dn = 0;
    for (uint32_t e = 0; e < n_experts; e++) {
        const qw6_hip_matrix_t* m[3] = {&gate[e], &up[e], &down[e]};
        for (int k = 0; k < 3; k++) {
            int f;
            if (!m[k]->data) return fail("expert %u matrix %d has no data", e, k);
            if (check_matrix(m[k]->quant, m[k]->rows, m[k]->cols, &f)) return -1;
            if (f < 0) return fail("expert %u matrix %d: F32 experts not supported", e, k);
            const uint32_t wr = k < 2 ? inter : hidden, wc = k < 2 ? hidden : inter;
            if (m[k]->rows != wr || m[k]->cols != wc)
                return fail("expert %u matrix %d shape %ux%u, expected %ux%u", e, k,
                            m[k]->rows, m[k]->cols, wr, wc);
            if ((uintptr_t)m[k]->data & 15u) return fail("expert %u matrix %d not 16-B aligned", e, k);
            tab[e].p[k] = (const uint8_t*)m[k]->data;
            tab[e].fmt[k] = f;
            tab[e].rb[k] = (m[k]->cols / 256) * fmt_block_bytes(f);
            (k < 2 ? mgu : mdn) |= fmt_table_mask(f);
            if (k < 2 && tab[e].rb[k] > rb_gu) rb_gu = tab[e].rb[k];
            if (k == 2 && tab[e].rb[k] > rb_dn) rb_dn = tab[e].rb[k];
        }
    }
    DevGuard g(c->device);
    qw6_hip_experts_t* E = new qw6_hip_experts_t();
    E->rb_gu_max = rb_gu;
    for (int k = 0; k < 3; k++) {   // expert e at base + e * stride, one format?
        PackRef& P = E->pk[k];
        P.base = tab[0].p[k];
        P.fmt = tab[0].fmt[k];
        P.rb = tab[0].rb[k];
        P.stride = n_experts > 1 ? (uint64_t)(tab[1].p[k] - tab[0].p[k]) : 0;
        P.regular = 1;
        for (uint32_t e = 0; e < n_experts && P.regular; e++)
            if (tab[e].fmt[k] != P.fmt ||
                tab[e].p[k] != tab[0].p[k] + P.stride * e || (P.stride & 15u))
                P.regular = 0;
    }
    E->fmt_gu = tab[0].fmt[0];
    E->fmt_dn = tab[0].fmt[2];
    E->xl_dn = tab[0].fmt[2];
    E->gu_same = 1;
    E->fmask_gu = E->fmask_dn = 0;
    for (uint32_t e = 0; e < n_experts; e++) {
        E->fmask_gu |= prefill_supports(tab[e].fmt[0]) ? 1u << tab[e].fmt[0] : 1u << 31;
        E->fmask_dn |= prefill_supports(tab[e].fmt[2]) ? 1u << tab[e].fmt[2] : 1u << 31;
        if (tab[e].fmt[0] != E->fmt_gu || tab[e].fmt[1] != E->fmt_gu) E->fmt_gu = -1;
        if (tab[e].fmt[2] != E->fmt_dn) E->fmt_dn = -1;
        if (E->xl_dn >= 0 && x_layout(tab[e].fmt[2]) != x_layout(E->xl_dn)) E->xl_dn = -1;
        if (tab[e].fmt[0] != tab[e].fmt[1]) E->gu_same = 0;
    }
    E->rb_dn_max = rb_dn;
    E->ctx = c;
    E->n = n_experts;
    E->hidden = hidden;
    E->inter = inter;
    E->tmask_gu = mgu;
    E->tmask_dn = mdn;
    if (hipMalloc((void**)&E->dev, sizeof(ExpertEnt) * n_experts) != hipSuccess ||
        hipMemcpy(E->dev, tab.data(), sizeof(ExpertEnt) * n_experts, hipMemcpyHostToDevice) !=
            hipSuccess) {
        if (E->dev) (void)hipFree(E->dev);
        delete E;
        return fail("expert table allocation failed");
    }
    *out = E;
    return 0;
}

void qw6_hip_experts_free(qw6_hip_experts_t* e) {
    if (!e) return;
    DevGuard g(e->ctx->device);
    (void)hipFree(e->dev);
    delete e;
}

}  // extern "C"

namespace {

int ensure_ws(qw6_hip_ctx_t* c, uint32_t hidden, uint32_t inter) {
    if (c->logits && c->ws_hidden >= hidden && c->ws_inter >= inter) return 0;
    hidden = hidden > c->ws_hidden ? hidden : c->ws_hidden;
    inter = inter > c->ws_inter ? inter : c->ws_inter;
    void* p;
    if (alloc_owned(c, (size_t)kSplitMaxTok * 256 * 4, &p)) return -1;
    c->logits = (float*)p;
    if (alloc_owned(c, kSplitMaxTok * 4, &p)) return -1;
    c->sw = (float*)p;
    if (alloc_owned(c, (size_t)kSplitMaxTok * hidden * 4, &p)) return -1;
    c->xn = (float*)p;
    if (alloc_owned(c, kSplitMaxTok * sizeof(SlotTable), &p)) return -1;
    c->slots = (SlotTable*)p;
    if (alloc_owned(c, (size_t)kMidRows * inter * 4, &p)) return -1;
    c->mid = (float*)p;
    c->ws_hidden = hidden;
    c->ws_inter = inter;
    return 0;
}

int ensure_mx_ws(qw6_hip_ctx_t* c, uint32_t hidden, uint32_t inter) {
    if (c->mxa && c->mx_hidden >= hidden && c->mx_inter >= inter) return 0;
    hidden = hidden > c->mx_hidden ? hidden : c->mx_hidden;
    inter = inter > c->mx_inter ? inter : c->mx_inter;
    void* p;
    if (alloc_owned(c, (size_t)(hidden / 32) * 64 * 16, &p)) return -1;
    c->mxa = (uint4*)p;
    if (alloc_owned(c, (size_t)(hidden / 256) * 192 * 2, &p)) return -1;
    c->mxs = (uint16_t*)p;
    if (alloc_owned(c, (size_t)(kMaxSlots + 1) * (inter / 32) * 64 * 16, &p)) return -1;
    c->mma = (uint4*)p;
    if (alloc_owned(c, (size_t)(kMaxSlots + 1) * (inter / 256) * 192 * 2, &p)) return -1;
    c->mms = (uint16_t*)p;
    c->mx_hidden = hidden;
    c->mx_inter = inter;
    return 0;
}

int ensure_prefill_ws(qw6_hip_ctx_t* c, uint32_t hidden, uint32_t inter, uint32_t n_experts,
                      uint32_t top_k) {
    (void)top_k;
    if (c->pre.ybuf && c->pre_hidden >= hidden && c->pre_inter >= inter &&
        c->pre_experts >= n_experts)
        return 0;
    const uint32_t T = c->max_tokens, K8 = 8;
    const size_t E = prefill_entries(T, K8);
    void* p;
    PrefillWs& w = c->pre;
    if (alloc_owned(c, (size_t)T * K8 * 4, &p)) return -1;
    w.pidx = (uint32_t*)p;
    if (alloc_owned(c, (size_t)T * K8 * 4, &p)) return -1;
    w.pw = (float*)p;
    if (alloc_owned(c, E * 4, &p)) return -1;
    w.ent_tok = (uint32_t*)p;
    if (alloc_owned(c, E * 4, &p)) return -1;
    w.ent_w = (float*)p;
    if (alloc_owned(c, (size_t)T * K8 * 4, &p)) return -1;
    w.ent_pos = (uint32_t*)p;
    if (alloc_owned(c, (size_t)prefill_tiles_max(T, K8, 256) * sizeof(uint4), &p)) return -1;
    w.tiles = (uint4*)p;
    if (alloc_owned(c, 16, &p)) return -1;
    w.n_tiles = (uint32_t*)p;
    if (alloc_owned(c, (size_t)2 * prefill_tiles_max(T, K8, 256) * 4, &p)) return -1;
    w.forder = (uint32_t*)p;
    if (alloc_owned(c, 2 * 8 * 2 * 4, &p)) return -1;
    w.fseg = (uint32_t*)p;
    if (alloc_owned(c, (size_t)T * 256 * 4, &p)) return -1;
    w.logits = (float*)p;
    if (alloc_owned(c, (size_t)T * hidden * 4, &p)) return -1;
    w.xn = (float*)p;
    for (int k = 0; k < 3; k++) {   // bf16 parts of the input and of mid
        if (alloc_owned(c, (size_t)T * hidden * 2, &p)) return -1;
        w.xp[k] = (uint16_t*)p;
        if (alloc_owned(c, E * inter * 2, &p)) return -1;
        w.mp[k] = (uint16_t*)p;
    }
    if (alloc_owned(c, (size_t)T * (hidden / 32) * 3 * 2, &p)) return -1;
    w.xs3 = (uint16_t*)p;
    if (alloc_owned(c, E * (inter / 32) * 3 * 2, &p)) return -1;
    w.ms3 = (uint16_t*)p;
    if (alloc_owned(c, E * hidden * 4, &p)) return -1;
    w.ybuf = (float*)p;
    c->pre_hidden = hidden;
    c->pre_inter = inter;
    c->pre_experts = n_experts;
    return 0;
}

// A kernel launch, timed by its own dispatch (hipExtLaunchKernel start/stop
// events, no extra queue packets) when ev is given.
template <typename... Args>
int launch_k(void (*kern)(Args...), uint32_t grid, uint32_t block, size_t lds, hipStream_t st,
             hipEvent_t* ev, const MoeArgs& a, uint32_t gy = 1) {
    if (ev) {
        void* args[] = {(void*)&a};
        CK(hipExtLaunchKernel((const void*)kern, dim3(grid, gy), dim3(block), args, lds, st, ev[0],
                              ev[1], 0));
    } else {
        kern<<<dim3(grid, gy), block, lds, st>>>(a);
        CK(hipGetLastError());
    }
    return 0;
}

struct MoeLaunch {
    bool router;             // k_moe_router runs
    bool mx;                 // the small-batch MFMA kernels (k_mx_*)
    uint32_t gy;             // grid rows of k_moe_gate_up1 / k_moe_down<1>: one per token
    uint32_t grid_r;
    uint32_t grid_b1;
    bool has_sh;             // the layer has a shared expert
    size_t lds_b1;
    int fg, fd;              // format of the gate/up (down) kernels, -1: mixed
    uint32_t mg, md;         // the formats present (bit f: format f), gate/up and down
    size_t lds_b, lds_c;
    uint32_t grid_b, grid_c, nw_b, nw_c;
};

// The format sets with their own instantiations of the mixed-format expert
// kernels (at the model's row length): the IQ2_M layer's, IQ2_XXS
// routed gate/up beside a Q4_K shared one, and IQ3_S / IQ2_S routed downs
// beside a Q6_K shared one. Other mixes take the six-format switch.
constexpr uint32_t kSetGateUpIq2m = (1u << F_Q4K) | (1u << F_IQ2XXS);
constexpr uint32_t kSetDownIq2m = (1u << F_Q6K) | (1u << F_IQ2S) | (1u << F_IQ3S);

// Run fn(IC<F>, IC<KU>) for the expert-kernel instantiation of format f
// (mask: the formats present) and KU = K/32 units per row: format- and
// size-specialised kernels at the model's row length KU_fast (one format, or
// the set above), the generic (six-format switch) kernel otherwise.
template <int KU_fast, uint32_t kSet, typename Fn>
void launch_expert_kernel(int f, uint32_t mask, uint32_t KU, Fn fn) {
    if (f >= 0 && KU == (uint32_t)KU_fast) {
        launch_by_fmt(f, 1, [&](auto, auto fc) { fn(fc, IC<KU_fast>{}); });
        return;
    }
    if (f < 0 && KU == (uint32_t)KU_fast && mask == kSet) {
        fn(IC<fmt_set(kSet)>{}, IC<KU_fast>{});
        return;
    }
    switch (KU) {
    case 8: fn(IC<-1>{}, IC<8>{}); break;
    case 16: fn(IC<-1>{}, IC<16>{}); break;
    case 32: fn(IC<-1>{}, IC<32>{}); break;
    default: fn(IC<-1>{}, IC<64>{}); break;
    }
}

int launch_moe(const MoeArgs& a, const MoeLaunch& m, hipStream_t st, hipEvent_t* ev) {
    if (m.router) {
        int rc = 0;
        auto by_nv = [&](auto tc) {
            constexpr int T = decltype(tc)::value;
            switch (a.hidden / 256) {
            case 1: rc = launch_k(k_moe_router<T, 1>, m.grid_r, 64, 0, st, ev, a); break;
            case 2: rc = launch_k(k_moe_router<T, 2>, m.grid_r, 64, 0, st, ev, a); break;
            case 4: rc = launch_k(k_moe_router<T, 4>, m.grid_r, 64, 0, st, ev, a); break;
            default: rc = launch_k(k_moe_router<T, 8>, m.grid_r, 64, 0, st, ev, a); break;
            }
        };
        auto by_nv_rows = [&]() {   // one token per grid row
            const uint32_t gx = (m.grid_r + 7u) & ~7u;
            constexpr uint32_t B = 64 * kRouterWaves;
            switch (a.hidden / 256) {
            case 1: rc = launch_k(k_moe_router<1, 1, true>, gx, 64, 0, st, ev, a, a.T); break;
            case 2: rc = launch_k(k_moe_router_w<2, kRouterWaves, true>, gx, B, 0, st, ev, a, a.T); break;
            case 4: rc = launch_k(k_moe_router_w<4, kRouterWaves, true>, gx, B, 0, st, ev, a, a.T); break;
            default: rc = launch_k(k_moe_router_w<8, kRouterWaves, true>, gx, B, 0, st, ev, a, a.T); break;
            }
        };
        if (!m.mx && a.T > 1) {   // the fp32 kernels' launches of several tokens
            by_nv_rows();
        } else if (!m.mx && a.hidden >= 512) {   // one token, kRouterWaves waves per router row
            switch (a.hidden / 256) {
            case 2: rc = launch_k(k_moe_router_w<2, kRouterWaves>, m.grid_r, 64 * kRouterWaves, 0, st, ev, a); break;
            case 4: rc = launch_k(k_moe_router_w<4, kRouterWaves>, m.grid_r, 64 * kRouterWaves, 0, st, ev, a); break;
            default: rc = launch_k(k_moe_router_w<8, kRouterWaves>, m.grid_r, 64 * kRouterWaves, 0, st, ev, a); break;
            }
        } else {
            switch (a.T) {
            case 1: by_nv(IC<1>{}); break;
            case 2: by_nv(IC<2>{}); break;
            case 3: by_nv(IC<3>{}); break;
            default: by_nv(IC<4>{}); break;
            }
        }
        if (rc) return rc;
    } else if (ev) {
        CK(hipEventRecord(ev[0], st));
        CK(hipEventRecord(ev[1], st));
    }
    int rc = 0;
    if (m.mx) {
        switch (a.T) {
        case 1: rc = launch_k(k_mx_gate_up<1>, m.grid_b, 64 * m.nw_b, m.lds_b, st, ev ? ev + 2 : nullptr, a); break;
        case 2: rc = launch_k(k_mx_gate_up<2>, m.grid_b, 64 * m.nw_b, m.lds_b, st, ev ? ev + 2 : nullptr, a); break;
        case 3: rc = launch_k(k_mx_gate_up<3>, m.grid_b, 64 * m.nw_b, m.lds_b, st, ev ? ev + 2 : nullptr, a); break;
        default: rc = launch_k(k_mx_gate_up<4>, m.grid_b, 64 * m.nw_b, m.lds_b, st, ev ? ev + 2 : nullptr, a); break;
        }
        if (rc) return rc;
        switch (a.T) {
        case 1: rc = launch_k(k_mx_down<1>, m.grid_c, 64 * m.nw_c, m.lds_c, st, ev ? ev + 4 : nullptr, a); break;
        case 2: rc = launch_k(k_mx_down<2>, m.grid_c, 64 * m.nw_c, m.lds_c, st, ev ? ev + 4 : nullptr, a); break;
        case 3: rc = launch_k(k_mx_down<3>, m.grid_c, 64 * m.nw_c, m.lds_c, st, ev ? ev + 4 : nullptr, a); break;
        default: rc = launch_k(k_mx_down<4>, m.grid_c, 64 * m.nw_c, m.lds_c, st, ev ? ev + 4 : nullptr, a); break;
        }
        return rc;
    }
    // the fp32 kernels; the multi-token instantiations (MT) read their
    // token's buffers by token_view
    auto fp32 = [&](auto mt) {
        constexpr bool MT = decltype(mt)::value;
        launch_expert_kernel<64, kSetGateUpIq2m>(m.fg, m.mg, a.hidden / 32, [&](auto fc, auto kc) {
            constexpr int F = decltype(fc)::value;
            const uint32_t nw = a.top_k + (m.has_sh ? gate_up1_shared_waves(MT, F) : 0u);
            rc = launch_k(k_moe_gate_up1<F, decltype(kc)::value, MT>, m.grid_b1, 64 * nw, m.lds_b1, st,
                          ev ? ev + 2 : nullptr, a, m.gy);
        });
        if (rc) return;
        launch_expert_kernel<16, kSetDownIq2m>(m.fd, m.md, a.inter / 32, [&](auto fc, auto kc) {
            rc = launch_k(k_moe_down<1, decltype(fc)::value, decltype(kc)::value, MT>, m.grid_c,
                          64 * m.nw_c, m.lds_c, st, ev ? ev + 4 : nullptr, a, m.gy);
        });
    };
    if (m.gy > 1) fp32(std::true_type{});
    else fp32(std::false_type{});
    return rc;
}

// qw6_hip_moe_forward and, with noalloc, qw6_hip_moe_forward_noalloc: the
// latter never takes the grouped kernels and runs the per-token ones on the
// static workspace instead of the context's.
int moe_forward_impl(qw6_hip_ctx_t* c, const qw6_hip_moe_layer_t* L, const float* x,
                     const float* logits, const float* residual, uint32_t n_tok, float* out,
                     uint32_t* idx, float* w, void* stream, bool noalloc) {
    if (!c || !L || !L->experts || !x || !out) return fail("null pointer");
    if (n_tok == 0) return 0;
    if (!noalloc && n_tok > c->max_tokens)
        return fail("n_tok %u > context max_tokens %u", n_tok, c->max_tokens);
    const qw6_hip_experts_t* E = L->experts;
    if (L->hidden != E->hidden || L->inter != E->inter)
        return fail("layer dims %ux%u do not match the expert table %ux%u", L->hidden, L->inter,
                    E->hidden, E->inter);
    if (!fast_k(L->hidden) || !fast_k(L->inter))
        return fail("decode MoE kernels need hidden and inter in {256, 512, 1024, 2048}");
    if (L->top_k == 0 || L->top_k > 8 || L->top_k > E->n) return fail("top_k %u out of range", L->top_k);
    if (!L->router && !logits) return fail("neither router nor logits given");
    if (((uintptr_t)L->router | (uintptr_t)x | (uintptr_t)out | (uintptr_t)L->shared_router |
         (uintptr_t)L->norm_w | (uintptr_t)residual) & 15u)
        return fail("router, shared_router, norm_w, x, residual and out must be 16-byte aligned");
    const bool has_sh = L->shared_gate.data != nullptr;
    MatD sg = {nullptr, 0, 0, 0, 0}, su = sg, sd = sg;
    uint32_t mgu = E->tmask_gu, mdn = E->tmask_dn;
    if (has_sh) {
        const qw6_hip_matrix_t* m[3] = {&L->shared_gate, &L->shared_up, &L->shared_down};
        MatD* d[3] = {&sg, &su, &sd};
        for (int k = 0; k < 3; k++) {
            int f;
            if (!m[k]->data) return fail("shared expert matrix %d missing", k);
            if (check_matrix(m[k]->quant, m[k]->rows, m[k]->cols, &f)) return -1;
            if (f < 0) return fail("F32 shared expert not supported");
            const uint32_t wr = k < 2 ? L->inter : L->hidden, wc = k < 2 ? L->hidden : L->inter;
            if (m[k]->rows != wr || m[k]->cols != wc) return fail("shared matrix %d shape", k);
            if ((uintptr_t)m[k]->data & 15u) return fail("shared matrix %d not 16-B aligned", k);
            *d[k] = {(const uint8_t*)m[k]->data, f, wr, wc, (wc / 256) * fmt_block_bytes(f)};
            (k < 2 ? mgu : mdn) |= fmt_table_mask(f);
        }
    } else if (L->shared_router) {
        return fail("shared_router given without a shared expert");
    }
    // every expert's gate and up share a format, so one unit layout serves both
    if (!E->gu_same || (has_sh && sg.fmt != su.fmt))
        return fail("gate and up of each expert must share a quant type");
    DevGuard g(c->device);
    hipStream_t st = (hipStream_t)stream;
    // batched tokens: grouped MFMA contraction when every expert matrix has a
    // format the grouped kernels decode; one launch per format present
    // (qw6_hip_set_mode: 0 automatic, 1 per-token, 2 grouped)
    const bool grouped_ok = !((E->fmask_gu | E->fmask_dn) >> 31) &&
                            (!has_sh || (prefill_supports(sg.fmt) && prefill_supports(sd.fmt))) &&
                            L->hidden % 256 == 0 && L->inter % 256 == 0;
    if (noalloc && c->mode == 2)
        return fail("the grouped MFMA path needs context workspace: not available without allocation");
    if (c->mode == 2 && !grouped_ok)
        return fail("grouped MFMA path: an expert matrix has a format the grouped kernels do not decode");
    const uint32_t min_grouped = (mgu | mdn) ? kGroupedMinTokensIq : kGroupedMinTokens;
    if (!noalloc && grouped_ok && (c->mode == 2 || (c->mode == 0 && n_tok >= min_grouped))) {
        if (ensure_prefill_ws(c, L->hidden, L->inter, E->n, L->top_k)) return -1;
        PrefillLayer P;
        memset(&P, 0, sizeof P);
        P.hidden = L->hidden; P.inter = L->inter; P.n_experts = E->n; P.top_k = L->top_k;
        P.T = n_tok;
        P.x = x; P.logits = logits; P.router = logits ? nullptr : L->router;
        P.shared_router = L->shared_router; P.norm_w = L->norm_w; P.norm_eps = L->norm_eps;
        P.residual = residual; P.out = out; P.idx_out = idx; P.w_out = w;
        P.experts = E->dev;
        for (int k = 0; k < 3; k++) P.pk[k] = E->pk[k];
        P.fmask_gu = E->fmask_gu; P.fmask_dn = E->fmask_dn;
        P.sg = sg; P.su = su; P.sd = sd;
        return prefill_forward(P, c->pre, st);
    }
    // per-token path: the fp32 kernels (k_moe_*) or the small-batch MFMA
    // kernels (k_mx_*: mode 3, or automatic for more than one token per launch)
    const bool mx_any = c->mode == 3;
    DecodeWs ws;
    if (noalloc) {
        const size_t need = carve_decode_ws(nullptr, L->hidden, L->inter, nullptr);
        if (need > kScratchBytes)
            return fail("layer %ux%u needs %zu bytes of decode workspace; the static workspace "
                        "holds %zu", L->hidden, L->inter, need, kScratchBytes);
        carve_decode_ws(c->scratch, L->hidden, L->inter, &ws);
    } else {
        if (ensure_ws(c, L->hidden, L->inter)) return -1;
        if (mx_any && ensure_mx_ws(c, L->hidden, L->inter)) return -1;
        ws = {c->logits, c->sw, c->xn, c->slots, c->mid, c->mxa, c->mxs, c->mma, c->mms};
    }

    MoeArgs a;
    memset(&a, 0, sizeof a);
    a.hidden = L->hidden;
    a.inter = L->inter;
    a.n_experts = E->n;
    a.top_k = L->top_k;
    a.shared_router = L->shared_router;
    a.norm_w = L->norm_w;
    a.norm_eps = L->norm_eps;
    a.experts = E->dev;
    for (int k = 0; k < 3; k++) a.pk[k] = E->pk[k];
    a.sg = sg; a.su = su; a.sd = sd;
    a.logits = ws.logits; a.sw = ws.sw; a.xn = ws.xn; a.mid = ws.mid; a.slots = ws.slots;
    a.tmask_gu = mgu;
    a.tmask_dn = mdn;
    a.xl_dn = E->xl_dn;
    a.xs = ws.mxs; a.ma = ws.mma; a.ms = ws.mms;
    // k_mx_* launch shape: the staged block of a format (largest of those in use)
    auto sb_of = [](int f) {
        if (f >= 0) return mx_stage_bytes(f);
        uint32_t b = 0;
        for (int k = 0; k < F_NFMT; k++) b = b > mx_stage_bytes(k) ? b : mx_stage_bytes(k);
        return b;
    };
    const uint32_t sb_gu = std::max(sb_of(E->fmt_gu), has_sh ? sb_of(sg.fmt) : 0u);
    const uint32_t sb_dn = std::max(sb_of(E->fmt_dn), has_sh ? sb_of(sd.fmt) : 0u);
    const uint32_t nkb_gu = L->hidden / 256, nkb_dn = L->inter / 256;
    // k_mx_gate_up: one wave per 256-column block, at least kMaxTok waves
    // (waves t < T route token t; the epilogue reads 128 threads' sums)
    const uint32_t mx_nw_b = std::max<uint32_t>(kMaxTok, nkb_gu < 8 ? nkb_gu : 8);
    const uint32_t mx_tab_gu = mx_tab(mgu).bytes, mx_tab_dn = mx_tab(mdn).bytes;
    a.mx_gu_soff = mx_tab_gu;
    a.mx_sb = sb_dn;

    MoeLaunch m;
    m.fg = (has_sh && sg.fmt != E->fmt_gu) ? -1 : E->fmt_gu;
    m.fd = (has_sh && sd.fmt != E->fmt_dn) ? -1 : E->fmt_dn;
    m.mg = (E->fmask_gu & ((1u << F_NFMT) - 1u)) | (has_sh ? 1u << sg.fmt : 0u);
    m.md = (E->fmask_dn & ((1u << F_NFMT) - 1u)) | (has_sh ? 1u << sd.fmt : 0u);
    const uint32_t rpsg = 64 / (L->hidden / 32), rpsd = 64 / (L->inter / 32);
    // k_moe_gate_up1: LDS pair slot of the widest (gate, up) step pair in use
    uint32_t pbb = has_sh ? fmt_block_bytes(sg.fmt) : 0u;   // widest block in use
    for (int f = 0; f < F_NFMT; f++)
        if (E->fmt_gu < 0 || E->fmt_gu == f) pbb = std::max(pbb, fmt_block_bytes(f));
    a.gu_pb = 16u * pbb;   // 8 blocks of gate and of up
    const uint32_t R_c = kStepsDn * rpsd;
    m.grid_c = (L->hidden + R_c - 1) / R_c;
    // the router kernel runs when it has work: the router GEMV (no logits
    // given), the shared-expert weight, or the input RMSNorm
    m.router = (!logits && L->router) || L->shared_router != nullptr || L->norm_w != nullptr;
    m.grid_r = E->n + (L->shared_router ? 1u : 0u);

    // The fp32 kernels (k_moe_gate_up1, k_moe_down<1>) take launches of up to
    // kSplitMaxTok tokens, one row of their grids per token (token_view);
    // mode 3 the small-batch MFMA kernels, launches of up to kMaxTok tokens.
    const bool mx = c->mode == 3;
    const uint32_t chunk = mx ? kMaxTok : kSplitMaxTok;
    // k_moe_gate_up1: one workgroup per kStepsGu row steps of every matrix
    // pair, kStepsGu LDS pair slots per matrix pair (the shared expert's
    // split over its waves)
    m.grid_b1 = (L->inter + kStepsGu * rpsg - 1) / (kStepsGu * rpsg);
    m.has_sh = has_sh;
    m.lds_b1 = (size_t)tab_bytes(mgu) + (size_t)(L->top_k + (has_sh ? 1u : 0u)) * kStepsGu * a.gu_pb;
    if (!mx && m.lds_b1 > kMxLdsBudget) return fail("gate/up tile exceeds the LDS budget");
    const uint32_t grid_c_valu = m.grid_c;
    for (uint32_t t0 = 0; t0 < n_tok; t0 += chunk) {
        const uint32_t T = n_tok - t0 < chunk ? n_tok - t0 : chunk;
        a.T = T;
        m.mx = mx;
        a.max_u = mx ? T * L->top_k : L->top_k;   // the fp32 kernels: per token
        a.xa = mx ? ws.mxa : nullptr;   // k_moe_router writes the operands
        m.gy = mx ? 1u : T;
        m.grid_c = grid_c_valu;
        a.x = x + (size_t)t0 * L->hidden;
        a.xin = L->norm_w ? ws.xn : a.x;
        a.router = logits ? nullptr : L->router;
        a.route_logits = logits ? logits + (size_t)t0 * E->n : ws.logits;
        a.residual = residual ? residual + (size_t)t0 * L->hidden : nullptr;
        a.out = out + (size_t)t0 * L->hidden;
        a.idx_out = idx ? idx + (size_t)t0 * L->top_k : nullptr;
        a.w_out = w ? w + (size_t)t0 * L->top_k : nullptr;
        const uint32_t ntot = a.max_u + (has_sh ? 1u : 0u);
        // k_moe_down: 9 waves (8 routed matrices + the shared one); 8 from 4
        // tokens on (3 for layers without IQ formats; one wave takes two
        // matrices), where 24 waves fit three workgroups per CU instead of two
        const uint32_t nw_dn = T >= 4 || (T == 3 && mdn == 0) ? 8u : down_waves<1>();
        m.nw_c = ntot < nw_dn ? ntot : nw_dn;
        m.lds_c = (size_t)tab_bytes(mdn) + (size_t)m.nw_c * kStepsDn * kSlotBytes +
                  (size_t)ntot * R_c * 4 + 16;
        if (!mx && m.lds_c > kLdsBudget) return fail("down tile exceeds the LDS budget");
        m.router = (!logits && L->router) || L->shared_router != nullptr || L->norm_w != nullptr;
        m.grid_r = E->n + (L->shared_router ? 1u : 0u);
        if (mx) {
            // gate/up: blocks of 16 rows, one wave per 256-column block (up to 8)
            const uint32_t nbw = (nkb_gu + mx_nw_b - 1) / mx_nw_b;
            a.n_sh_wg = has_sh ? L->inter / 16 : 0u;
            m.grid_b = a.n_sh_wg + a.max_u * (L->inter / 16);
            m.nw_b = mx_nw_b;
            m.lds_b = (size_t)mx_tab_gu + (size_t)mx_nw_b * nbw * 2 * sb_gu;
            // down: blocks of 16 rows, the (matrix, 256-column block) pairs
            // staged a round at a time
            const uint32_t npair = ntot * nkb_dn;
            const uint32_t fixed = mx_tab_dn + npair * 256u;   // tables + per-pair sums
            if (fixed + sb_dn > kMxLdsBudget) return fail("small-batch down tile exceeds the LDS budget");
            a.mx_nsl = std::min(npair, (kMxLdsBudget - fixed) / sb_dn);
            m.grid_c = L->hidden / 16;
            m.nw_c = npair < 16 ? npair : 16;
            m.lds_c = (size_t)fixed + (size_t)a.mx_nsl * sb_dn;
            // the router kernel always runs: it writes the input operands
            m.router = true;
            m.grid_r = std::max(m.grid_r, L->hidden / 32);
            if (m.lds_b > kMxLdsBudget) return fail("small-batch gate/up tile exceeds the LDS budget");
        }
        hipEvent_t* ev = nullptr;
        if (c->prof_calls < c->prof_cap) ev = &c->prof_ev[kProfEv * c->prof_calls++];
        const int rc = launch_moe(a, m, st, ev);
        if (rc) return rc;
    }
    return 0;
}

}  // namespace

extern "C" {

int qw6_hip_moe_forward(qw6_hip_ctx_t* c, const qw6_hip_moe_layer_t* L, const float* x,
                        const float* logits, const float* residual, uint32_t n_tok,
                        float* out, uint32_t* idx, float* w, void* stream) {
    return moe_forward_impl(c, L, x, logits, residual, n_tok, out, idx, w, stream, false);
}

int qw6_hip_moe_forward_noalloc(qw6_hip_ctx_t* c, const qw6_hip_moe_layer_t* L,
                                const float* x, const float* logits, const float* residual,
                                uint32_t n_tok, float* out, uint32_t* idx, float* w,
                                void* stream) {
    return moe_forward_impl(c, L, x, logits, residual, n_tok, out, idx, w, stream, true);
}

int qw6_hip_profile(qw6_hip_ctx_t* c, uint32_t max_calls) {
    if (!c) return fail("null ctx");
    DevGuard g(c->device);
    for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
    c->prof_ev.clear();
    c->prof_cap = c->prof_calls = 0;
    if (max_calls == 0) return 0;
    c->prof_ev.resize(kProfEv * (size_t)max_calls);
    for (auto& e : c->prof_ev) CK(hipEventCreate(&e));
    c->prof_cap = max_calls;
    return 0;
}

int qw6_hip_profile_read(qw6_hip_ctx_t* c, float ms[3], uint32_t* calls) {
    if (!c || !ms || !calls) return fail("null pointer");
    DevGuard g(c->device);
    for (int k = 0; k < 3; k++) ms[k] = 0.f;
    for (uint32_t i = 0; i < c->prof_calls; i++) {
        CK(hipEventSynchronize(c->prof_ev[kProfEv * i + kProfEv - 1]));
        for (int k = 0; k < 3; k++) {
            float t = 0.f;
            CK(hipEventElapsedTime(&t, c->prof_ev[kProfEv * i + 2 * k],
                                   c->prof_ev[kProfEv * i + 2 * k + 1]));
            ms[k] += t;
        }
    }
    *calls = c->prof_calls;
    return 0;
}

int qw6_hip_argmax_host(const float* x, uint32_t n, uint32_t* out_idx, float* out_val) {
    if (!x || !out_idx) return fail("null pointer");
    if (n == 0) return fail("argmax of an empty vector");
    DevBuf bx, bp, bo;
    CK(hipMalloc(&bx.p, (size_t)n * 4));
    CK(hipMalloc(&bp.p, (size_t)kArgmaxBlocks * 8));
    CK(hipMalloc(&bo.p, 4));
    CK(hipMemcpy(bx.p, x, (size_t)n * 4, hipMemcpyHostToDevice));
    if (launch_argmax((const float*)bx.p, n, (uint64_t*)bp.p, (uint32_t*)bo.p, nullptr)) return -1;
    CK(hipDeviceSynchronize());
    uint32_t i = 0;
    CK(hipMemcpy(&i, bo.p, 4, hipMemcpyDeviceToHost));
    if (i >= n) return fail("argmax index %u out of range", i);
    *out_idx = i;
    if (out_val) *out_val = x[i];   // the selected element itself, bit for bit
    return 0;
}

int qw6_hip_sampling_greedy_host(const float* logits, uint32_t n, uint32_t* token) {
    if (!logits || !token) return fail("null pointer");
    return qw6_hip_argmax_host(logits, n, token, nullptr);
}

int qw6_hip_argmax(qw6_hip_ctx_t* c, const float* x, uint32_t n, uint32_t* out, void* stream) {
    if (!c || !x || !out) return fail("null pointer");
    if (n == 0) return fail("argmax of an empty vector");
    DevGuard g(c->device);
    if (ensure_argmax_ws(c)) return -1;
    return launch_argmax(x, n, c->amax_part, out, (hipStream_t)stream);
}

int qw6_hip_output_greedy(qw6_hip_ctx_t* c, const qw6_hip_matrix_t* w, const float* x,
                          const float* norm_w, float eps, float* logits, uint32_t* token,
                          void* stream) {
    if (!c || !w || !w->data || !x || !logits || !token) return fail("null pointer");
    int f;
    if (check_matrix(w->quant, w->rows, w->cols, &f)) return -1;
    if ((uintptr_t)w->data & 15u) return fail("weight data not 16-byte aligned");
    // the head kernels read x and the norm weight in 16-byte pieces
    if (((uintptr_t)x | (uintptr_t)norm_w) & 15u) return fail("x and norm_w must be 16-byte aligned");
    DevGuard g(c->device);
    const hipStream_t st = (hipStream_t)stream;
    if (ensure_argmax_ws(c)) return -1;
    const uint32_t rb = w->quant == 0 ? w->cols * 4 : (w->cols / 256) * fmt_block_bytes(f);
    const MatD W = {(const uint8_t*)w->data, w->quant == 0 ? -1 : f, w->rows, w->cols, rb};
    const int hr = launch_head(W, x, norm_w, eps, logits, c->amax_part, token, st);
    if (hr <= 0) return hr;   // else: a shape the streaming pass does not take
    const float* xin = x;
    if (norm_w) {   // final RMSNorm (qw6.c:2490-2492)
        if (!c->head_x || c->head_hidden < w->cols) {
            void* p;
            if (alloc_owned(c, (size_t)w->cols * 4, &p)) return -1;
            c->head_x = (float*)p;
            c->head_hidden = w->cols;
        }
        k_rmsnorm<<<1, kWG, 0, st>>>(x, norm_w, c->head_x, w->cols, eps);
        CK(hipGetLastError());
        xin = c->head_x;
    }
    if (launch_matvec(W, xin, logits, 1, st)) return -1;   // qw6.c:2493
    return launch_argmax(logits, w->rows, c->amax_part, token, st);
}

int qw6_hip_rmsnorm(qw6_hip_ctx_t* c, const float* x, const float* w, float* y, uint32_t n,
                    uint32_t n_tok, float eps, void* stream) {
    if (!c || !x || !w || !y) return fail("null pointer");
    if (n == 0 || n_tok == 0) return fail("empty rmsnorm");
    DevGuard g(c->device);
    k_rmsnorm<<<n_tok, kWG, 0, (hipStream_t)stream>>>(x, w, y, n, eps);
    CK(hipGetLastError());
    return 0;
}

int qw6_hip_synth_blocks(void* dst, int32_t quant, uint64_t nblocks, uint64_t first,
                         uint64_t seed, uint64_t stream_id, void* stream) {
    if (!dst) return fail("null pointer");
    const int f = fmt_of_quant(quant);
    if (f < 0) return fail("unsupported quant %d", quant);
    if (nblocks == 0) return 0;
    const uint64_t key = sm_stream_key(seed, stream_id);
    const uint64_t nb = (nblocks + 255) / 256;
    if (nb > 0x7fffffffull) return fail("too many blocks");
    k_synth_blocks<<<(uint32_t)nb, 256, 0, (hipStream_t)stream>>>(
        (uint8_t*)dst, f, nblocks, first, key, fmt_block_bytes(f));
    CK(hipGetLastError());
    return 0;
}

int qw6_hip_synth_normal(float* dst, uint64_t n, float mean, float sd, uint64_t seed,
                         uint64_t stream_id, void* stream) {
    if (!dst) return fail("null pointer");
    if (n == 0) return 0;
    const uint64_t key = sm_stream_key(seed, stream_id);
    const uint64_t nb = (n + 255) / 256;
    if (nb > 0x7fffffffull) return fail("too many values");
    k_synth_normal<<<(uint32_t)nb, 256, 0, (hipStream_t)stream>>>(dst, n, mean, sd, key);
    CK(hipGetLastError());
    return 0;
}

}  // extern "C"
