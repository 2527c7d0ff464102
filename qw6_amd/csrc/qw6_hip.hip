// qw6_hip.hip -- gfx950 kernels and C ABI of the routed-expert MoE FFN path.
//
// Decode path (fp32 accumulation), three kernels per MoE layer:
//   moe_router : router GEMV over all experts; the last workgroup to finish
//                (device-scope counter) runs the softmax top-k for every token
//                and builds the list of distinct selected experts ("slots");
//                extra workgroups run the shared expert's gate/up/SiLU, which
//                does not depend on routing.
//   moe_gate_up: one workgroup per (slot, row tile): stages the tile's gate
//                and up rows into LDS with direct-to-LDS 16-byte loads, then
//                dequantizes in registers and writes silu(gate) * up.
//   moe_down   : one workgroup per tile of output rows, over all slots plus the
//                shared expert in a fixed order, gate-weighted combine (and
//                residual) in registers -- no atomics, deterministic.
// Routing never leaves the device (qw6's Vulkan path reads idx/w back to the
// host per layer, qw6_vk.c:3371-3374).
//
// Lane mapping: a row of K columns has U = K/32 units of 32 weights
// (qw6_dev.h); a wave covers 64/U rows per step, lane -> (row, unit) fixed,
// so each lane keeps its unit's activations in registers across rows.

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "../../include/qw6_hip.h"
#include "qw6_dev.h"

using namespace qw6;

namespace {

__device__ const IqTables g_tabs = make_tables();

constexpr int kWG = 256;           // threads per workgroup (4 waves)
constexpr uint32_t kMaxTok = 4;    // tokens per decode launch
constexpr uint32_t kLdsBudget = 64 * 1024;

thread_local char g_err[512];

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "qw6_hip: %s\n", g_err);
    return -1;
}

#define CK(expr)                                                                   \
    do {                                                                           \
        hipError_t _e = (expr);                                                    \
        if (_e != hipSuccess)                                                      \
            return fail("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),    \
                        __FILE__, __LINE__);                                       \
    } while (0)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// ---- staging: global bytes -> LDS ----------------------------------------------

// Copy `bytes` (even) from 16-byte-aligned global src to 16-byte-aligned LDS
// dst with all threads of the workgroup: 16-byte direct-to-LDS loads for the
// body, 2-byte copies for the tail. The caller waits (stage_wait) before use.
__device__ __forceinline__ void stage(uint8_t* dst, const uint8_t* src, uint32_t bytes) {
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    const uint32_t n16 = bytes >> 4;
    for (uint32_t c0 = 0; c0 < n16; c0 += kWG) {
        const uint32_t wbase = c0 + wave * 64;
        if (wbase < n16) {
            const uint32_t c = c0 + tid;
            if (c < n16)
                __builtin_amdgcn_global_load_lds((glb_void_t*)(src + 16ull * c),
                                                 (lds_void_t*)(dst + 16u * wbase), 16, 0, 0);
        }
    }
    const uint32_t rem = (bytes & 15u) >> 1;
    if (tid < rem) {
        const uint16_t v = ((const uint16_t*)(src + 16ull * n16))[tid];
        ((uint16_t*)(dst + 16u * n16))[tid] = v;
    }
}

__device__ __forceinline__ void stage_wait() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

// Lattice tables needed by `mask` into LDS (IqTables layout at tab).
__device__ __forceinline__ void stage_tables(uint8_t* tab, uint32_t mask) {
    const uint8_t* g = (const uint8_t*)&g_tabs;
    if (mask & 1u) stage(tab + kTabOffIq2xxs, g + kTabOffIq2xxs, 256 * 8);
    if (mask & 2u) stage(tab + kTabOffIq2s, g + kTabOffIq2s, 1024 * 8);
    if (mask & 4u) stage(tab + kTabOffIq3s, g + kTabOffIq3s, 512 * 4);
}

__host__ __device__ inline uint32_t tab_bytes(uint32_t mask) {
    return mask & 4u ? kTabBytes : mask & 2u ? kTabOffIq3s : mask & 1u ? kTabOffIq2s : 0u;
}

// ---- one matrix tile: per-row dot products --------------------------------------

struct MatD {
    const uint8_t* p;
    int32_t fmt;
    uint32_t rows, cols, rb;   // rb: bytes per row
};

// Rows [0, rows_valid) of a tile staged at LDS word pointer `tile`; wave w
// processes steps s: local row = (w*steps + s)*rps + lane/U. emit(row, acc)
// is called on the first lane of each row group.
template <int T, typename Emit>
__device__ __forceinline__ void tile_rows(int f, const uint32_t* lds, uint32_t tile_off,
                                          uint32_t rb, uint32_t K, const float* x,
                                          uint32_t ldx, const uint32_t* tab,
                                          uint32_t rows_valid, uint32_t steps, Emit emit) {
    const uint32_t U = K >> 5, rps = 64 / U;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t unit = lane & (U - 1), blk = unit >> 3;
    const int j = (int)(unit & 7);
    const uint32_t bb = fmt_block_bytes(f);
    float xr[T][32], sx[T][4];
#pragma unroll
    for (int t = 0; t < T; t++) load_unit_x(f, x + (size_t)t * ldx, blk, j, xr[t], sx[t]);
    for (uint32_t s = 0; s < steps; s++) {
        const uint32_t rl = (wave * steps + s) * rps + lane / U;
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = 0.f;
        if (rl < rows_valid) unit_dot<T>(f, lds, tile_off + rl * rb + blk * bb, j, tab, xr, sx, acc);
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = group_sum(acc[t], U);
        if (unit == 0 && rl < rows_valid) emit(rl, acc);
    }
}

// ---- single-matrix matvec --------------------------------------------------------

template <int T>
__global__ __launch_bounds__(kWG) void k_matvec(MatD W, const float* __restrict__ x,
                                                float* __restrict__ y, uint32_t R,
                                                uint32_t steps, uint32_t tmask) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t r0 = blockIdx.x * R;
    const uint32_t nv = min(R, W.rows - r0);
    const uint32_t toff = tab_bytes(tmask);
    stage_tables(smem, tmask);
    stage(smem + toff, W.p + (size_t)r0 * W.rb, nv * W.rb);
    stage_wait();
    const uint32_t* s = (const uint32_t*)smem;
    tile_rows<T>(W.fmt, s, toff, W.rb, W.cols, x, W.cols, s, nv, steps,
                 [&](uint32_t rl, const float(&acc)[T]) {
#pragma unroll
                     for (int t = 0; t < T; t++) y[(size_t)t * W.rows + r0 + rl] = acc[t];
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
    // 64-thread workgroup: reuse the 256-thread staging with idle upper chunks.
    const uint32_t lane = threadIdx.x;
    const uint8_t* src = W.p + (size_t)r * W.rb;
    const uint8_t* g = (const uint8_t*)&g_tabs;
    for (uint32_t c = lane; c < toff / 16; c += 64)
        ((uint4*)smem)[c] = ((const uint4*)g)[c];
    for (uint32_t c = lane; c < W.rb / 2; c += 64)
        ((uint16_t*)(smem + toff))[c] = ((const uint16_t*)src)[c];
    __syncthreads();
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
        for (int t = 0; t < T; t++) load_unit_x(W.fmt, x + (size_t)t * W.cols, blk, j, xr[t], sx[t]);
        unit_dot<T>(W.fmt, s, toff + blk * bb, j, s, xr, sx, acc);
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float v = group_sum(acc[t], 64);
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
        const float v = group_sum(acc[t], 64);
        if (lane == 0) y[(size_t)t * rows + r] = v;
    }
}

// ---- routing ---------------------------------------------------------------------

// One wave: top_k rounds of (max value, lowest index), selected set to -inf,
// then softmax over the selected values in selection order
// (qw6_cpu_moe_route, qw6.c:2796-2827). Lane 0 writes idx/w.
__device__ void wave_route(const float* logits, uint32_t n, uint32_t top_k, uint32_t* idx,
                           float* w) {
    const uint32_t lane = threadIdx.x & 63;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t e = lane + 64u * i;
        v[i] = e < n ? logits[e] : -INFINITY;
    }
    float sel[8];
    uint32_t sid[8];
    for (uint32_t k = 0; k < top_k; k++) {
        float bv = v[0];
        uint32_t bi = lane < n ? lane : 0xffffffffu;
#pragma unroll
        for (int i = 1; i < 4; i++) {
            const uint32_t e = lane + 64u * i;
            if (e < n && (v[i] > bv || bi == 0xffffffffu)) { bv = v[i]; bi = e; }
        }
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const uint32_t oi = (uint32_t)__shfl_xor((int)bi, m, 64);
            if (oi != 0xffffffffu &&
                (bi == 0xffffffffu || ov > bv || (ov == bv && oi < bi) ||
                 (!(ov == ov) && !(bv == bv) && oi < bi))) {
                bv = ov; bi = oi;
            }
        }
        sel[k] = bv;
        sid[k] = bi;
        if ((bi & 63u) == lane) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (lane + 64u * i == bi) v[i] = -INFINITY;
        }
    }
    if (lane == 0) {
        float mx = sel[0];
        for (uint32_t k = 1; k < top_k; k++) mx = sel[k] > mx ? sel[k] : mx;
        float e[8], sum = 0.f;
        for (uint32_t k = 0; k < top_k; k++) { e[k] = expf(sel[k] - mx); sum += e[k]; }
        for (uint32_t k = 0; k < top_k; k++) { idx[k] = sid[k]; w[k] = e[k] / sum; }
    }
}

__global__ __launch_bounds__(64) void k_route(const float* __restrict__ logits, uint32_t n,
                                              uint32_t top_k, uint32_t* idx, float* w) {
    const uint32_t t = blockIdx.x;
    wave_route(logits + (size_t)t * n, n, top_k, idx + t * top_k, w + t * top_k);
}

// ---- MoE decode kernels --------------------------------------------------------------

struct ExpertEnt {            // device expert table entry
    const uint8_t* p[3];      // gate, up, down
    int32_t fmt[3];
    uint32_t rb[3];
};

struct MoeArgs {
    uint32_t hidden, inter, n_experts, top_k, T, max_u;
    const float* x;
    const float* router;
    const float* logits_in;
    const float* shared_router;
    const ExpertEnt* experts;
    MatD sg, su, sd;          // shared expert; sg.p == nullptr: none
    float* logits;            // [T][n_experts]
    uint32_t* idx;            // [T][top_k]
    float* w;                 // [T][top_k]
    uint32_t* nslots;         // [1]
    uint32_t* slot_e;         // [max_u] expert of each slot
    float* wt;                // [max_u][T] gate weight of slot u for token t
    float* sw;                // [T] shared weight
    float* mid;               // [(max_u + 1)][T][inter], shared at max_u
    uint32_t* counter;
    const float* residual;
    float* out;
    uint32_t* idx_out;
    float* w_out;
    uint32_t n_router_wg, rr_per_wg;     // router workgroups, rows per router WG
    uint32_t rb_tile, rb_steps;          // gate/up tile rows and steps per wave
    uint32_t rc_tile, rc_steps;          // down tile rows and steps per wave
    uint32_t tmask_gu, tmask_dn;
};

// gate/up/silu for rows [r0, r0+R) of one expert -> mid[T][inter].
template <int T>
__device__ void gate_up_tile(const MatD& G, const MatD& Up, uint32_t r0, uint32_t R,
                             uint32_t steps, const float* x, uint32_t hidden, float* mid,
                             uint32_t inter, uint32_t tmask, uint8_t* smem) {
    const uint32_t nv = min(R, G.rows - r0);
    const uint32_t toff = tab_bytes(tmask);
    const uint32_t gbytes = (nv * G.rb + 15u) & ~15u;
    float* gv = (float*)(smem + toff + gbytes + ((nv * Up.rb + 15u) & ~15u) + 16);   // [R][T]
    stage_tables(smem, tmask);
    stage(smem + toff, G.p + (size_t)r0 * G.rb, nv * G.rb);
    stage(smem + toff + gbytes, Up.p + (size_t)r0 * Up.rb, nv * Up.rb);
    stage_wait();
    const uint32_t* s = (const uint32_t*)smem;
    tile_rows<T>(G.fmt, s, toff, G.rb, hidden, x, hidden, s, nv, steps,
                 [&](uint32_t rl, const float(&acc)[T]) {
#pragma unroll
                     for (int t = 0; t < T; t++) gv[rl * T + t] = acc[t];
                 });
    __syncthreads();
    tile_rows<T>(Up.fmt, s, toff + gbytes, Up.rb, hidden, x, hidden, s, nv, steps,
                 [&](uint32_t rl, const float(&acc)[T]) {
#pragma unroll
                     for (int t = 0; t < T; t++) {
                         const float g = gv[rl * T + t];
                         mid[(size_t)t * inter + r0 + rl] = g / (1.0f + expf(-g)) * acc[t];
                     }
                 });
}

template <int T>
__global__ __launch_bounds__(kWG) void k_moe_router(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t b = blockIdx.x;
    if (b >= a.n_router_wg) {   // shared expert gate/up
        const uint32_t tile = b - a.n_router_wg;
        gate_up_tile<T>(a.sg, a.su, tile * a.rb_tile, a.rb_tile, a.rb_steps, a.x, a.hidden,
                        a.mid + (size_t)a.max_u * T * a.inter, a.inter, a.tmask_gu, smem);
        return;
    }
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t e0 = b * a.rr_per_wg, e1 = min(e0 + a.rr_per_wg, a.n_experts);
    if (a.router) {
        for (uint32_t e = e0 + wave; e < e1; e += 4) {
            const float4* wr = (const float4*)(a.router + (size_t)e * a.hidden);
            float acc[T];
#pragma unroll
            for (int t = 0; t < T; t++) acc[t] = 0.f;
            for (uint32_t c = lane; c < a.hidden / 4; c += 64) {
                const float4 wv = wr[c];
#pragma unroll
                for (int t = 0; t < T; t++) {
                    const float4 xv = ((const float4*)(a.x + (size_t)t * a.hidden))[c];
                    acc[t] = fmaf(wv.x, xv.x, acc[t]);
                    acc[t] = fmaf(wv.y, xv.y, acc[t]);
                    acc[t] = fmaf(wv.z, xv.z, acc[t]);
                    acc[t] = fmaf(wv.w, xv.w, acc[t]);
                }
            }
#pragma unroll
            for (int t = 0; t < T; t++) {
                const float v = group_sum(acc[t], 64);
                if (lane == 0) a.logits[(size_t)t * a.n_experts + e] = v;
            }
        }
    } else {
        for (uint32_t i = threadIdx.x; i < (e1 - e0) * T; i += kWG) {
            const uint32_t t = i / (e1 - e0), e = e0 + i % (e1 - e0);
            a.logits[(size_t)t * a.n_experts + e] = a.logits_in[(size_t)t * a.n_experts + e];
        }
    }
    // Last router workgroup to finish routes every token.
    __shared__ uint32_t s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(a.counter, 1u) == a.n_router_wg - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (uint32_t t = wave; t < T; t += 4) {
        wave_route(a.logits + (size_t)t * a.n_experts, a.n_experts, a.top_k,
                   a.idx + t * a.top_k, a.w + t * a.top_k);
        if (a.shared_router) {
            float acc = 0.f;
            for (uint32_t c = lane; c < a.hidden; c += 64)
                acc = fmaf(a.shared_router[c], a.x[(size_t)t * a.hidden + c], acc);
            acc = group_sum(acc, 64);
            if (lane == 0) a.sw[t] = 1.0f / (1.0f + expf(-acc));
        } else if (lane == 0) {
            a.sw[t] = 1.0f;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t n = 0;
        for (uint32_t t = 0; t < T; t++)
            for (uint32_t k = 0; k < a.top_k; k++) {
                const uint32_t e = a.idx[t * a.top_k + k];
                uint32_t u = 0;
                while (u < n && a.slot_e[u] != e) u++;
                if (u == n) {
                    a.slot_e[n] = e;
                    for (uint32_t tt = 0; tt < T; tt++) a.wt[n * T + tt] = 0.f;
                    n++;
                }
                a.wt[u * T + t] = a.w[t * a.top_k + k];
                if (a.idx_out) a.idx_out[t * a.top_k + k] = e;
                if (a.w_out) a.w_out[t * a.top_k + k] = a.w[t * a.top_k + k];
            }
        *a.nslots = n;
        *a.counter = 0u;
    }
}

template <int T>
__global__ __launch_bounds__(kWG) void k_moe_gate_up(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t ntile = (a.inter + a.rb_tile - 1) / a.rb_tile;
    const uint32_t u = blockIdx.x / ntile, tile = blockIdx.x % ntile;
    if (u >= *a.nslots) return;
    const ExpertEnt& E = a.experts[a.slot_e[u]];
    const MatD G = {E.p[0], E.fmt[0], a.inter, a.hidden, E.rb[0]};
    const MatD Up = {E.p[1], E.fmt[1], a.inter, a.hidden, E.rb[1]};
    gate_up_tile<T>(G, Up, tile * a.rb_tile, a.rb_tile, a.rb_steps, a.x, a.hidden,
                    a.mid + (size_t)u * T * a.inter, a.inter, a.tmask_gu, smem);
}

constexpr uint32_t kMaxSteps = 4;

template <int T>
__global__ __launch_bounds__(kWG) void k_moe_down(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t r0 = blockIdx.x * a.rc_tile;
    const uint32_t nv = min(a.rc_tile, a.hidden - r0);
    const uint32_t nslot = *a.nslots;
    const bool has_sh = a.sd.p != nullptr;
    const uint32_t ntot = nslot + (has_sh ? 1u : 0u);
    const uint32_t toff = tab_bytes(a.tmask_dn);
    const uint32_t* s = (const uint32_t*)smem;
    const uint32_t U = a.inter >> 5, rps = 64 / U;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t unit = lane & (U - 1), blk = unit >> 3;
    const int j = (int)(unit & 7);
    float acc_out[kMaxSteps][T], shv[kMaxSteps][T];
#pragma unroll
    for (uint32_t q = 0; q < kMaxSteps; q++)
#pragma unroll
        for (int t = 0; t < T; t++) { acc_out[q][t] = 0.f; shv[q][t] = 0.f; }
    // slot u < nslot: routed expert a.slot_e[u]; slot nslot: the shared expert
    auto slot_mat = [&](uint32_t u) -> MatD {
        if (u < nslot) {
            const ExpertEnt& E = a.experts[a.slot_e[u]];
            return MatD{E.p[2], E.fmt[2], a.hidden, a.inter, E.rb[2]};
        }
        return a.sd;
    };
    stage_tables(smem, a.tmask_dn);
    // Slots in batches that fit the LDS budget, all rows of a batch in flight.
    uint32_t u0 = 0;
    while (u0 < ntot) {
        uint32_t off = toff, u1 = u0;
        while (u1 < ntot) {
            const MatD D = slot_mat(u1);
            const uint32_t bytes = (nv * D.rb + 15u) & ~15u;
            if (u1 > u0 && off + bytes + 16 > kLdsBudget) break;
            stage(smem + off, D.p + (size_t)r0 * D.rb, nv * D.rb);
            off += bytes;
            u1++;
        }
        stage_wait();
        off = toff;
        for (uint32_t u = u0; u < u1; u++) {
            const MatD D = slot_mat(u);
            const bool shared = u >= nslot;
            const float* xm = a.mid + (size_t)(shared ? a.max_u : u) * T * a.inter;
            float wts[T];
#pragma unroll
            for (int t = 0; t < T; t++) wts[t] = shared ? 0.f : a.wt[u * T + t];
            const uint32_t bb = fmt_block_bytes(D.fmt);
            float xr[T][32], sx[T][4];
#pragma unroll
            for (int t = 0; t < T; t++)
                load_unit_x(D.fmt, xm + (size_t)t * a.inter, blk, j, xr[t], sx[t]);
#pragma unroll
            for (uint32_t q = 0; q < kMaxSteps; q++) {
                if (q >= a.rc_steps) break;
                const uint32_t rl = (wave * a.rc_steps + q) * rps + lane / U;
                float acc[T];
#pragma unroll
                for (int t = 0; t < T; t++) acc[t] = 0.f;
                if (rl < nv) unit_dot<T>(D.fmt, s, off + rl * D.rb + blk * bb, j, s, xr, sx, acc);
#pragma unroll
                for (int t = 0; t < T; t++) {
                    const float v = group_sum(acc[t], U);
                    if (shared) shv[q][t] = v;
                    else acc_out[q][t] = fmaf(wts[t], v, acc_out[q][t]);
                }
            }
            off += (nv * D.rb + 15u) & ~15u;
        }
        __syncthreads();
        u0 = u1;
    }
    if (unit != 0) return;
#pragma unroll
    for (uint32_t q = 0; q < kMaxSteps; q++) {
        if (q >= a.rc_steps) break;
        const uint32_t rl = (wave * a.rc_steps + q) * rps + lane / U;
        if (rl >= nv) continue;
#pragma unroll
        for (int t = 0; t < T; t++) {
            float v = acc_out[q][t];
            if (has_sh) v = fmaf(a.sw[t], shv[q][t], v);
            if (a.residual) v += a.residual[(size_t)t * a.hidden + r0 + rl];
            a.out[(size_t)t * a.hidden + r0 + rl] = v;
        }
    }
}

// ---- small elementwise kernels ---------------------------------------------------

__global__ void k_silu_mul(const float* g, const float* u, float* o, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
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
    ss = group_sum(ss, 64);
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
    const float z = sm_normal(key, 3 * i) * sd;
    dst[i] = mean == 0.f ? z : mean + z;
}

}  // namespace

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
    uint32_t* idx;
    float* w;
    uint32_t* nslots;
    uint32_t* slot_e;
    float* wt;
    float* sw;
    float* mid;
    uint32_t* counter;
    uint32_t ws_experts, ws_inter, ws_topk;
    // per-kernel timing (qw6_hip_profile)
    std::vector<hipEvent_t> prof_ev;
    uint32_t prof_cap, prof_calls;
};

struct qw6_hip_experts_s {
    qw6_hip_ctx_t* ctx;
    ExpertEnt* dev;
    uint32_t n;
    uint32_t hidden, inter;
    uint32_t tmask_gu, tmask_dn;
    uint32_t rb_gu_max;   // widest gate/up row in bytes
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

uint32_t min_rows_align(uint32_t rb) {   // rows r such that r * rb % 16 == 0
    uint32_t r = 1;
    while ((r * rb) & 15u) r <<= 1;
    return r;
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
            const uint32_t toff = tmask & 4u ? kTabBytes : tmask & 2u ? kTabOffIq3s
                                : tmask & 1u ? kTabOffIq2s : 0u;
            if (fast_k(W.cols)) {
                const uint32_t U = W.cols / 32, rps = 64 / U;
                uint32_t steps = 1;
                while (steps < kMaxSteps && 4 * rps * steps * 2 * W.rb <= 32768) steps <<= 1;
                uint32_t R = 4 * rps * steps;
                while (R % min_rows_align(W.rb)) { steps <<= 1; R = 4 * rps * steps; }
                const size_t lds = toff + R * W.rb + 32;
                const dim3 grid((W.rows + R - 1) / R);
                switch (T) {
                case 1: k_matvec<1><<<grid, kWG, lds, st>>>(W, xt, yt, R, steps, tmask); break;
                case 2: k_matvec<2><<<grid, kWG, lds, st>>>(W, xt, yt, R, steps, tmask); break;
                case 3: k_matvec<3><<<grid, kWG, lds, st>>>(W, xt, yt, R, steps, tmask); break;
                default: k_matvec<4><<<grid, kWG, lds, st>>>(W, xt, yt, R, steps, tmask); break;
                }
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

}  // namespace

extern "C" {

const char* qw6_hip_last_error(void) { return g_err; }

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
    qw6_hip_ctx_t* c = new qw6_hip_ctx_t();
    c->device = device;
    c->max_tokens = max_tokens;
    c->mode = 0;
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
    if (!c || mode < 0 || mode > 2) return fail("bad mode");
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
    uint32_t mgu = 0, mdn = 0, rb_gu = 0;
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
        }
    }
    DevGuard g(c->device);
    qw6_hip_experts_t* E = new qw6_hip_experts_t();
    E->rb_gu_max = rb_gu;
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

int ensure_ws(qw6_hip_ctx_t* c, uint32_t n_experts, uint32_t inter, uint32_t top_k) {
    if (c->logits && c->ws_experts >= n_experts && c->ws_inter >= inter && c->ws_topk >= top_k)
        return 0;
    const uint32_t T = kMaxTok, max_u = T * 8;
    n_experts = n_experts > 256 ? n_experts : 256;
    inter = inter > c->ws_inter ? inter : c->ws_inter;
    void* p;
    if (alloc_owned(c, (size_t)T * n_experts * 4, &p)) return -1;
    c->logits = (float*)p;
    if (alloc_owned(c, (size_t)T * 8 * 4, &p)) return -1;
    c->idx = (uint32_t*)p;
    if (alloc_owned(c, (size_t)T * 8 * 4, &p)) return -1;
    c->w = (float*)p;
    if (alloc_owned(c, 16, &p)) return -1;
    c->nslots = (uint32_t*)p;
    if (alloc_owned(c, max_u * 4, &p)) return -1;
    c->slot_e = (uint32_t*)p;
    if (alloc_owned(c, (size_t)max_u * T * 4, &p)) return -1;
    c->wt = (float*)p;
    if (alloc_owned(c, T * 4, &p)) return -1;
    c->sw = (float*)p;
    if (alloc_owned(c, (size_t)(max_u + 1) * T * inter * 4, &p)) return -1;
    c->mid = (float*)p;
    if (alloc_owned(c, 256, &p)) return -1;
    c->counter = (uint32_t*)p;
    c->ws_experts = n_experts;
    c->ws_inter = inter;
    c->ws_topk = 8;
    return 0;
}

template <int T>
int launch_moe_T(const MoeArgs& a, size_t lds_r, uint32_t grid_r, size_t lds_b,
                        uint32_t grid_b, size_t lds_c, uint32_t grid_c, hipStream_t st,
                        hipEvent_t* ev) {
    if (ev) CK(hipEventRecord(ev[0], st));
    k_moe_router<T><<<grid_r, kWG, lds_r, st>>>(a);
    CK(hipGetLastError());
    if (ev) CK(hipEventRecord(ev[1], st));
    k_moe_gate_up<T><<<grid_b, kWG, lds_b, st>>>(a);
    CK(hipGetLastError());
    if (ev) CK(hipEventRecord(ev[2], st));
    k_moe_down<T><<<grid_c, kWG, lds_c, st>>>(a);
    CK(hipGetLastError());
    if (ev) CK(hipEventRecord(ev[3], st));
    return 0;
}

}  // namespace

extern "C" {

int qw6_hip_moe_forward(qw6_hip_ctx_t* c, const qw6_hip_moe_layer_t* L, const float* x,
                        const float* logits, const float* residual, uint32_t n_tok,
                        float* out, uint32_t* idx, float* w, void* stream) {
    if (!c || !L || !L->experts || !x || !out) return fail("null pointer");
    if (n_tok == 0) return 0;
    if (n_tok > c->max_tokens) return fail("n_tok %u > context max_tokens %u", n_tok, c->max_tokens);
    const qw6_hip_experts_t* E = L->experts;
    if (L->hidden != E->hidden || L->inter != E->inter)
        return fail("layer dims %ux%u do not match the expert table %ux%u", L->hidden, L->inter,
                    E->hidden, E->inter);
    if (!fast_k(L->hidden) || !fast_k(L->inter))
        return fail("decode MoE kernels need hidden and inter in {256, 512, 1024, 2048}");
    if (L->top_k == 0 || L->top_k > 8 || L->top_k > E->n) return fail("top_k %u out of range", L->top_k);
    if (!L->router && !logits) return fail("neither router nor logits given");
    if (((uintptr_t)L->router | (uintptr_t)x | (uintptr_t)out) & 15u)
        return fail("router, x and out must be 16-byte aligned");
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
            *d[k] = {(const uint8_t*)m[k]->data, f, wr, wc, (wc / 256) * fmt_block_bytes(f)};
            (k < 2 ? mgu : mdn) |= fmt_table_mask(f);
        }
    }
    DevGuard g(c->device);
    if (ensure_ws(c, E->n, L->inter, L->top_k)) return -1;
    hipStream_t st = (hipStream_t)stream;

    MoeArgs a;
    memset(&a, 0, sizeof a);
    a.hidden = L->hidden;
    a.inter = L->inter;
    a.n_experts = E->n;
    a.top_k = L->top_k;
    a.router = L->router;
    a.shared_router = L->shared_router;
    a.experts = E->dev;
    a.sg = sg; a.su = su; a.sd = sd;
    a.logits = c->logits; a.idx = c->idx; a.w = c->w; a.nslots = c->nslots;
    a.slot_e = c->slot_e; a.wt = c->wt; a.sw = c->sw; a.mid = c->mid; a.counter = c->counter;
    a.tmask_gu = mgu;
    a.tmask_dn = mdn;
    // gate/up tiles: 4 waves x steps x (64/U) rows
    const uint32_t Ug = L->hidden / 32, rpsg = 64 / Ug;
    a.rb_steps = rpsg >= 4 ? 1 : 4 / rpsg;
    a.rb_tile = 4 * rpsg * a.rb_steps;
    const uint32_t Ud = L->inter / 32, rpsd = 64 / Ud;
    a.rc_steps = rpsd >= 4 ? 1 : 4 / rpsd;
    a.rc_tile = 4 * rpsd * a.rc_steps;
    a.rr_per_wg = L->router ? 4 : E->n;
    a.n_router_wg = (E->n + a.rr_per_wg - 1) / a.rr_per_wg;
    uint32_t rb_max = E->rb_gu_max;
    if (has_sh) rb_max = sg.rb > rb_max ? sg.rb : rb_max, rb_max = su.rb > rb_max ? su.rb : rb_max;
    auto gu_lds = [&]() {
        return (size_t)tab_bytes(mgu) + 2 * ((size_t)a.rb_tile * rb_max + 16) +
               a.rb_tile * kMaxTok * 4 + 64;
    };
    while (gu_lds() > kLdsBudget && a.rb_steps > 1) {
        a.rb_steps >>= 1;
        a.rb_tile = 4 * rpsg * a.rb_steps;
    }
    const size_t lds_gu = gu_lds();
    const uint32_t nsh_tiles = has_sh ? (L->inter + a.rb_tile - 1) / a.rb_tile : 0;
    const uint32_t ntile_b = (L->inter + a.rb_tile - 1) / a.rb_tile;
    const uint32_t grid_c = (L->hidden + a.rc_tile - 1) / a.rc_tile;
    if (lds_gu > kLdsBudget) return fail("gate/up tile exceeds LDS budget");

    for (uint32_t t0 = 0; t0 < n_tok; t0 += kMaxTok) {
        const uint32_t T = n_tok - t0 < kMaxTok ? n_tok - t0 : kMaxTok;
        a.T = T;
        a.max_u = T * L->top_k;
        a.x = x + (size_t)t0 * L->hidden;
        a.logits_in = logits ? logits + (size_t)t0 * E->n : nullptr;
        a.router = logits ? nullptr : L->router;
        a.rr_per_wg = a.router ? 4 : E->n;
        a.n_router_wg = (E->n + a.rr_per_wg - 1) / a.rr_per_wg;
        a.residual = residual ? residual + (size_t)t0 * L->hidden : nullptr;
        a.out = out + (size_t)t0 * L->hidden;
        a.idx_out = idx ? idx + (size_t)t0 * L->top_k : nullptr;
        a.w_out = w ? w + (size_t)t0 * L->top_k : nullptr;
        const uint32_t grid_r = a.n_router_wg + nsh_tiles;
        const uint32_t grid_b = a.max_u * ntile_b;
        hipEvent_t* ev = nullptr;
        if (c->prof_calls < c->prof_cap) ev = &c->prof_ev[4 * c->prof_calls++];
        int rc;
        switch (T) {
        case 1: rc = launch_moe_T<1>(a, lds_gu, grid_r, lds_gu, grid_b, kLdsBudget, grid_c, st, ev); break;
        case 2: rc = launch_moe_T<2>(a, lds_gu, grid_r, lds_gu, grid_b, kLdsBudget, grid_c, st, ev); break;
        case 3: rc = launch_moe_T<3>(a, lds_gu, grid_r, lds_gu, grid_b, kLdsBudget, grid_c, st, ev); break;
        default: rc = launch_moe_T<4>(a, lds_gu, grid_r, lds_gu, grid_b, kLdsBudget, grid_c, st, ev); break;
        }
        if (rc) return rc;
    }
    return 0;
}

int qw6_hip_profile(qw6_hip_ctx_t* c, uint32_t max_calls) {
    if (!c) return fail("null ctx");
    DevGuard g(c->device);
    for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
    c->prof_ev.clear();
    c->prof_cap = c->prof_calls = 0;
    if (max_calls == 0) return 0;
    c->prof_ev.resize(4 * (size_t)max_calls);
    for (auto& e : c->prof_ev) CK(hipEventCreate(&e));
    c->prof_cap = max_calls;
    return 0;
}

int qw6_hip_profile_read(qw6_hip_ctx_t* c, float ms[3], uint32_t* calls) {
    if (!c || !ms || !calls) return fail("null pointer");
    DevGuard g(c->device);
    ms[0] = ms[1] = ms[2] = 0.f;
    for (uint32_t i = 0; i < c->prof_calls; i++) {
        CK(hipEventSynchronize(c->prof_ev[4 * i + 3]));
        for (int k = 0; k < 3; k++) {
            float t = 0.f;
            CK(hipEventElapsedTime(&t, c->prof_ev[4 * i + k], c->prof_ev[4 * i + k + 1]));
            ms[k] += t;
        }
    }
    *calls = c->prof_calls;
    return 0;
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
