// qw6_prefill.hip -- the MoE FFN for a batch of tokens (prefill, batched
// verification) as grouped bf16-MFMA contractions on gfx950.
//
// qw6 runs its MoE block token by token (qw6_forward_token -> qw6_apply_layer_
// moe, qw6.c:2226-2290; qw6_prefill, qw6.c:2867-2882). With T tokens of top-8
// routing, expert e sees M_e of them; its gate/up/down are then T x K by K x N
// products over the M_e gathered rows. Kernels, in stream order:
//   k_pre_route   one wave per token: softmax top-k (wave_route), the
//                 shared-expert weight, the shared entries.
//   k_pre_sort    one workgroup: counting sort of the (token, k) pairs by
//                 expert into "entries", and a tile list of <= 32 entries of
//                 one expert (the shared expert last, with every token).
//   k_pre_gemm<0> gate and up for 64 intermediate rows of one tile:
//                 mid[entry] = silu(x.gate) * (x.up).
//   k_pre_gemm<1> down for 128 hidden rows of one tile, times the entry's
//                 gate weight -> ybuf[entry].
//   k_pre_combine out[t] = sum_k ybuf[entry(t, k)] + ybuf[shared entry(t)]
//                 (+ residual), a fixed order: deterministic, no atomics.
//
// Numerics of the contraction (rel-L2 ~1e-5 against the fp32 CPU path):
//  - weights enter the MFMA as their integer codes, exact in bf16: 128 + q
//    for a 4/5/6-bit code q (the byte pair {q, 0x43} is bf16 128 + q, one
//    v_perm per two codes);
//  - activations enter as bf16 hi + lo (hi = bf16(x), lo = bf16(x - hi)), two
//    MFMAs per 32-column sub-block;
//  - the fp32 sub-block scale d*sc multiplies each sub-block's 16x16 MFMA
//    result; the code bias (128 or 160) and the K-quant minimum dmin*m, both
//    of the form (per-row integer) x (per-token sub-block sum of x), are two
//    more small MFMAs per 256-column block with the sub-block sums as A.
// Sub-blocks are 32 columns in every format handled here (Q4_K, Q5_K, and
// Q6_K under qw6's even-scale rule, qw6.c:1567-1570).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw6_dev.h"
#include "qw6_moe.h"

namespace qw6 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kPM = 32;      // entries per tile (2 MFMA row groups of 16)
constexpr uint32_t kPWG = 256;    // threads per workgroup (4 waves)
constexpr uint32_t kRaw = 128;    // weight rows staged per workgroup and block

__host__ __device__ constexpr uint32_t raw_chunks(int f) {   // 16-B chunks per staged row block
    return (fmt_block_bytes(f) + 14 + 15) / 16;
}

// ---- routing -----------------------------------------------------------------------

// One wave per token t: routing, the shared-expert weight, the shared entry.
__global__ __launch_bounds__(64) void k_pre_route(PrefillLayer L, PrefillWs ws,
                                                  const float* __restrict__ xin,
                                                  const float* __restrict__ logits) {
    __shared__ uint2 scr[40];
    const uint32_t t = blockIdx.x, lane = threadIdx.x;
    wave_route(logits + (size_t)t * L.n_experts, L.n_experts, L.top_k, scr,
               ws.pidx + (size_t)t * L.top_k, ws.pw + (size_t)t * L.top_k);
    __builtin_amdgcn_wave_barrier();
    if (lane < L.top_k) {
        const size_t i = (size_t)t * L.top_k + lane;
        if (L.idx_out) L.idx_out[i] = ws.pidx[i];
        if (L.w_out) L.w_out[i] = ws.pw[i];
    }
    float sw = 1.0f;
    if (L.shared_router) {   // sigmoid(shared_router . x) (qw6.c:2267-2285)
        float acc = 0.f;
        const float* xr = xin + (size_t)t * L.hidden;
        for (uint32_t c = lane; c < L.hidden; c += 64) acc = fmaf(L.shared_router[c], xr[c], acc);
        acc = group_sum<64>(acc);
        sw = 1.0f / (1.0f + expf(-acc));
    }
    if (lane == 0) {
        const uint32_t e = L.T * L.top_k + t;
        ws.ent_tok[e] = t;
        ws.ent_w[e] = sw;
    }
}

// Counting sort of the T * top_k (token, k) pairs by expert, one workgroup.
// Entries of one expert are contiguous; their order inside the expert does
// not affect any result (every entry's output depends on its own row only,
// and the combine sums in (token, k) order).
__global__ __launch_bounds__(1024) void k_pre_sort(PrefillLayer L, PrefillWs ws) {
    __shared__ uint32_t cnt[257], off[257], cur[257], tof[257];
    const uint32_t tid = threadIdx.x;
    const uint32_t ne = L.T * L.top_k, E = L.n_experts;
    for (uint32_t e = tid; e <= E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < ne; i += blockDim.x) atomicAdd(&cnt[ws.pidx[i]], 1u);
    __syncthreads();
    if (tid < 64) {   // exclusive scans of the counts and of the tiles per expert
        uint32_t run = 0, trun = 0;
        for (uint32_t e0 = 0; e0 < E; e0 += 64) {
            const uint32_t e = e0 + tid;
            const uint32_t c = e < E ? cnt[e] : 0u;
            const uint32_t nt = (c + kPM - 1) / kPM;
            uint32_t sc = c, st = nt;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {   // inclusive wave scan
                const uint32_t oc = __shfl_up(sc, d), ot = __shfl_up(st, d);
                if (tid >= (uint32_t)d) { sc += oc; st += ot; }
            }
            if (e < E) { off[e] = run + sc - c; tof[e] = trun + st - nt; }
            run += __shfl(sc, 63);
            trun += __shfl(st, 63);
        }
        if (tid == 0) { off[E] = run; tof[E] = trun; }
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += blockDim.x) cur[e] = off[e];
    __syncthreads();
    for (uint32_t i = tid; i < ne; i += blockDim.x) {
        const uint32_t e = ws.pidx[i];
        const uint32_t pos = atomicAdd(&cur[e], 1u);
        ws.ent_tok[pos] = i / L.top_k;
        ws.ent_w[pos] = ws.pw[i];
        ws.ent_pos[i] = pos;
    }
    for (uint32_t e = tid; e < E; e += blockDim.x) {
        const uint32_t c = cnt[e];
        for (uint32_t j = 0; j * kPM < c; j++)
            ws.tiles[tof[e] + j] = make_uint4(e, off[e] + j * kPM, min(kPM, c - j * kPM), 0u);
    }
    const uint32_t nrt = tof[E];
    const uint32_t nsh = L.sg.p ? (L.T + kPM - 1) / kPM : 0u;
    for (uint32_t j = tid; j < nsh; j += blockDim.x)
        ws.tiles[nrt + j] = make_uint4(E, ne + j * kPM, min(kPM, L.T - j * kPM), 0u);
    if (tid == 0) *ws.n_tiles = nrt + nsh;
}

// ---- the grouped contraction --------------------------------------------------------

__device__ __forceinline__ uint4 u4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return make_uint4(a, b, c, d);
}
// Byte pairs {b0, 0x43}, {b1, 0x43} of the low half (hi = 0) or {b2,..}, {b3,..}
// (hi = 1) of w: bf16 values 128 + b.
__device__ __forceinline__ uint32_t codes2(uint32_t w, int hi) {
    return __builtin_amdgcn_perm(0x43434343u, w, hi ? 0x04030402u : 0x04010400u);
}
// Eight codes 128 + byte of (w0, w1) in MFMA operand order.
__device__ __forceinline__ uint4 codes8(uint32_t w0, uint32_t w1) {
    return u4(codes2(w0, 0), codes2(w0, 1), codes2(w1, 0), codes2(w1, 1));
}
__device__ __forceinline__ uint32_t bf16_bits(float f) {   // exact for the small integers used here
    return __float_as_uint(f) >> 16;
}
__device__ __forceinline__ f32x4 mfma(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// The B operands of one 16-row tile for one 256-column block, decoded from
// the raw block bytes in LDS (s = LDS words, R = byte offset of this lane's
// row block). Lane (n = l % 16, q = l / 16) holds codes of row n, columns
// 32 s + 8 q .. + 8 for the eight sub-blocks s, the fp32 sub-block scales of
// row n, and, in lanes q == 0, the per-sub-block integer factors of the
// bias / minimum terms as B operands over k = sub-block.
struct BTile {
    uint4 b[8];       // codes per sub-block
    float dsc[8];     // d * sc per sub-block
    uint4 bsc, bmin;  // B operands: sub-block scales, sub-block minimums (q == 0 lanes)
    float d, dmin;
};

template <int F>
__device__ __forceinline__ void decode_btile(const uint32_t* s, uint32_t R, uint32_t q,
                                             BTile& bt) {
    if (F == F_Q4K || F == F_Q5K) {
        bt.d = h2f(lds16(s, R));
        bt.dmin = h2f(lds16(s, R + 2));
        const uint32_t A = lds32(s, R + 4), B = lds32(s, R + 8), C = lds32(s, R + 12);
        uint32_t sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {   // qw6_get_scale_min_k4 (qw6.c:1480-1490)
            sc[j] = (A >> (8 * j)) & 63u;
            mn[j] = (B >> (8 * j)) & 63u;
            sc[j + 4] = ((C >> (8 * j)) & 15u) | (((A >> (8 * j + 6)) & 3u) << 4);
            mn[j + 4] = ((C >> (8 * j + 4)) & 15u) | (((B >> (8 * j + 6)) & 3u) << 4);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) bt.dsc[j] = bt.d * (float)sc[j];
        const uint32_t qo = F == F_Q4K ? 16u : 48u;   // qs offset
        uint32_t h0 = 0, h1 = 0;
        if (F == F_Q5K) { h0 = lds32(s, R + 16 + 8 * q); h1 = lds32(s, R + 20 + 8 * q); }
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint32_t w0 = lds32(s, R + qo + 32 * g + 8 * q);
            const uint32_t w1 = lds32(s, R + qo + 32 * g + 8 * q + 4);
            uint32_t l0 = w0 & 0x0f0f0f0fu, l1 = w1 & 0x0f0f0f0fu;
            uint32_t u0 = (w0 >> 4) & 0x0f0f0f0fu, u1 = (w1 >> 4) & 0x0f0f0f0fu;
            if (F == F_Q5K) {
                l0 |= ((h0 >> (2 * g)) & 0x01010101u) << 4;
                l1 |= ((h1 >> (2 * g)) & 0x01010101u) << 4;
                u0 |= ((h0 >> (2 * g + 1)) & 0x01010101u) << 4;
                u1 |= ((h1 >> (2 * g + 1)) & 0x01010101u) << 4;
            }
            bt.b[2 * g] = codes8(l0, l1);
            bt.b[2 * g + 1] = codes8(u0, u1);
        }
        bt.bsc = q == 0 ? u4(bf16_bits((float)sc[0]) | (bf16_bits((float)sc[1]) << 16),
                             bf16_bits((float)sc[2]) | (bf16_bits((float)sc[3]) << 16),
                             bf16_bits((float)sc[4]) | (bf16_bits((float)sc[5]) << 16),
                             bf16_bits((float)sc[6]) | (bf16_bits((float)sc[7]) << 16))
                        : u4(0, 0, 0, 0);
        bt.bmin = q == 0 ? u4(bf16_bits((float)mn[0]) | (bf16_bits((float)mn[1]) << 16),
                              bf16_bits((float)mn[2]) | (bf16_bits((float)mn[3]) << 16),
                              bf16_bits((float)mn[4]) | (bf16_bits((float)mn[5]) << 16),
                              bf16_bits((float)mn[6]) | (bf16_bits((float)mn[7]) << 16))
                         : u4(0, 0, 0, 0);
    } else {   // Q6_K: sub-block s = 4h + k, scale sc[8h + 2k] (qw6.c:1550-1578)
        bt.d = h2f(lds16(s, R + 208));
        bt.dmin = 0.f;
        float scf[8];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t sw0 = lds32(s, R + 192 + 8 * h), sw1 = lds32(s, R + 196 + 8 * h);
            scf[4 * h + 0] = (float)(int8_t)(sw0 & 0xffu);
            scf[4 * h + 1] = (float)(int8_t)((sw0 >> 16) & 0xffu);
            scf[4 * h + 2] = (float)(int8_t)(sw1 & 0xffu);
            scf[4 * h + 3] = (float)(int8_t)((sw1 >> 16) & 0xffu);
            const uint32_t a0 = lds32(s, R + 64 * h + 8 * q), a1 = lds32(s, R + 64 * h + 8 * q + 4);
            const uint32_t b0 = lds32(s, R + 64 * h + 32 + 8 * q), b1 = lds32(s, R + 64 * h + 36 + 8 * q);
            const uint32_t x0 = lds32(s, R + 128 + 32 * h + 8 * q), x1 = lds32(s, R + 132 + 32 * h + 8 * q);
            bt.b[4 * h + 0] = codes8((a0 & 0x0f0f0f0fu) | ((x0 & 0x03030303u) << 4),
                                     (a1 & 0x0f0f0f0fu) | ((x1 & 0x03030303u) << 4));
            bt.b[4 * h + 1] = codes8((b0 & 0x0f0f0f0fu) | (((x0 >> 2) & 0x03030303u) << 4),
                                     (b1 & 0x0f0f0f0fu) | (((x1 >> 2) & 0x03030303u) << 4));
            bt.b[4 * h + 2] = codes8(((a0 >> 4) & 0x0f0f0f0fu) | (((x0 >> 4) & 0x03030303u) << 4),
                                     ((a1 >> 4) & 0x0f0f0f0fu) | (((x1 >> 4) & 0x03030303u) << 4));
            bt.b[4 * h + 3] = codes8(((b0 >> 4) & 0x0f0f0f0fu) | (((x0 >> 6) & 0x03030303u) << 4),
                                     ((b1 >> 4) & 0x0f0f0f0fu) | (((x1 >> 6) & 0x03030303u) << 4));
        }
#pragma unroll
        for (int j = 0; j < 8; j++) bt.dsc[j] = bt.d * scf[j];
        bt.bsc = q == 0 ? u4(bf16_bits(scf[0]) | (bf16_bits(scf[1]) << 16),
                             bf16_bits(scf[2]) | (bf16_bits(scf[3]) << 16),
                             bf16_bits(scf[4]) | (bf16_bits(scf[5]) << 16),
                             bf16_bits(scf[6]) | (bf16_bits(scf[7]) << 16))
                        : u4(0, 0, 0, 0);
        bt.bmin = u4(0, 0, 0, 0);
    }
}

// Shared memory of k_pre_gemm.
struct GemmLds {
    uint4 a[2][8][2][64];        // A operands [row group][sub-block][hi, lo][lane]
    float sx[kPM][8];            // sum over each sub-block of (hi + lo)
    uint32_t raw[1];             // kRaw rows x raw_chunks(F) x 16 B, staged block bytes
};

// MODE 0: gate/up of 64 intermediate rows; MODE 1: down of 128 hidden rows.
// Block (tile, row group). Wave w: row tiles {2w, 2w+1} of 16 rows (MODE 0:
// gate and up rows 16w .. 16w+15 of the group; MODE 1: rows 32w .. 32w+31).
template <int MODE, int F>
__global__ __launch_bounds__(kPWG) void k_pre_gemm(PrefillLayer L, PrefillWs ws) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    GemmLds& S = *(GemmLds*)smem;
    const uint4 tile = ws.tiles[blockIdx.x < *ws.n_tiles ? blockIdx.x : 0];
    if (blockIdx.x >= *ws.n_tiles) return;
    const uint32_t mid_e = tile.x, ent0 = tile.y, cnt = tile.z;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t n = lane & 15u, q = lane >> 4;
    const bool shared = mid_e == L.n_experts;
    const uint32_t K = MODE == 0 ? L.hidden : L.inter;
    const uint32_t nblk = K / 256;
    constexpr uint32_t NCH = raw_chunks(F);
    constexpr uint32_t bb = fmt_block_bytes(F);
    const uint32_t rb = (K / 256) * bb;
    // weight rows of this workgroup: raw row rr -> matrix, row
    const uint32_t r0 = blockIdx.y * (MODE == 0 ? 64u : 128u);
    const uint8_t* m0;
    const uint8_t* m1 = nullptr;
    if (MODE == 0) {
        m0 = shared ? L.sg.p : L.pk[0].regular ? L.pk[0].base + L.pk[0].stride * mid_e
                                               : L.experts[mid_e].p[0];
        m1 = shared ? L.su.p : L.pk[1].regular ? L.pk[1].base + L.pk[1].stride * mid_e
                                               : L.experts[mid_e].p[1];
    } else {
        m0 = shared ? L.sd.p : L.pk[2].regular ? L.pk[2].base + L.pk[2].stride * mid_e
                                               : L.experts[mid_e].p[2];
    }
    auto row_ptr = [&](uint32_t rr) -> const uint8_t* {
        if (MODE == 0) return rr < 64 ? m0 + (size_t)(r0 + rr) * rb : m1 + (size_t)(r0 + rr - 64) * rb;
        return m0 + (size_t)(r0 + rr) * rb;
    };
    // this lane's two row tiles (raw rows)
    uint32_t rrow[2];
    if (MODE == 0) { rrow[0] = 16 * wave + n; rrow[1] = 64 + 16 * wave + n; }
    else { rrow[0] = 32 * wave + n; rrow[1] = 32 * wave + 16 + n; }
    const uint32_t bias = F == F_Q6K ? 160u : 128u;
    const uint32_t ngrp = (cnt + 15) / 16;   // 16-entry row groups in use

    f32x4 acc[2][2];
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
        for (int r = 0; r < 2; r++) acc[g][r] = f32x4{0.f, 0.f, 0.f, 0.f};

    // activation rows handled by this thread during staging
    const uint32_t am = tid >> 3, ac = tid & 7u;
    const float* arow = nullptr;
    if (am < cnt) {
        const uint32_t e = ent0 + am;
        arow = MODE == 0 ? L.x + (size_t)ws.ent_tok[e] * L.hidden : ws.mid + (size_t)e * L.inter;
    }

    for (uint32_t kb = 0; kb < nblk; kb++) {
        // stage the raw block bytes of the 128 rows (16-B chunks from the
        // aligned start of each row block)
        for (uint32_t c0 = wave * 64; c0 < kRaw * NCH; c0 += kPWG) {
            const uint32_t c = c0 + lane;
            const uint32_t rr = c / NCH, ch = c % NCH;
            const uint8_t* p = row_ptr(rr) + (size_t)kb * bb;
            const uint32_t off = (uint32_t)((uintptr_t)p & 15u);
            const uint8_t* pa = p - off + 16 * ch;
            if (16 * ch < off + bb)   // only chunks holding bytes of this row block
                __builtin_amdgcn_global_load_lds((glb_void_t*)pa,
                                                 (lds_void_t*)((uint8_t*)S.raw + 16u * c0), 16, 0, 0);
        }
        // activations: thread (am, ac) converts sub-block ac of entry am
        if (arow) {
            const float4* src = (const float4*)(arow + kb * 256 + 32 * ac);
            float v[32];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t4 = src[i];
                v[4 * i] = t4.x; v[4 * i + 1] = t4.y; v[4 * i + 2] = t4.z; v[4 * i + 3] = t4.w;
            }
            float sum = 0.f;
#pragma unroll
            for (uint32_t qq = 0; qq < 4; qq++) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float x0 = v[8 * qq + 2 * i], x1 = v[8 * qq + 2 * i + 1];
                    const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
                    const float r0f = x0 - (float)h0, r1f = x1 - (float)h1;
                    const __bf16 l0 = (__bf16)r0f, l1 = (__bf16)r1f;
                    sum += ((float)h0 + (float)l0) + ((float)h1 + (float)l1);
                    hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                    lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                }
                const uint32_t ln = (am & 15u) + 16u * qq;
                S.a[am >> 4][ac][0][ln] = u4(hw[0], hw[1], hw[2], hw[3]);
                S.a[am >> 4][ac][1][ln] = u4(lw[0], lw[1], lw[2], lw[3]);
            }
            S.sx[am][ac] = sum;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // B operands of this wave's two row tiles
        BTile bt[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint32_t R = rrow[r] * NCH * 16 + ((uintptr_t)(row_ptr(rrow[r]) + (size_t)kb * bb) & 15u);
            decode_btile<F>(S.raw, R, q, bt[r]);
        }
        // contraction
        for (uint32_t g = 0; g < ngrp; g++) {
            // A operands of the sub-block sums (k = sub-block, lanes q == 0) in
            // three bf16 parts: they multiply integer scales whose products
            // cancel the code bias, so they carry fp32 precision
            uint4 sx3[3] = {u4(0, 0, 0, 0), u4(0, 0, 0, 0), u4(0, 0, 0, 0)};
            if (q == 0) {
                uint32_t w3[3][4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t h[3][2];
#pragma unroll
                    for (int e2 = 0; e2 < 2; e2++) {
                        float r = S.sx[16 * g + n][2 * i + e2];
#pragma unroll
                        for (int p3 = 0; p3 < 3; p3++) {
                            const __bf16 b = (__bf16)r;
                            h[p3][e2] = (uint32_t)__builtin_bit_cast(uint16_t, b);
                            r -= (float)b;
                        }
                    }
#pragma unroll
                    for (int p3 = 0; p3 < 3; p3++) w3[p3][i] = h[p3][0] | (h[p3][1] << 16);
                }
#pragma unroll
                for (int p3 = 0; p3 < 3; p3++) sx3[p3] = u4(w3[p3][0], w3[p3][1], w3[p3][2], w3[p3][3]);
            }
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {
                const uint4 ah = S.a[g][sb][0][lane], al = S.a[g][sb][1][lane];
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    f32x4 c = mfma(ah, bt[r].b[sb], f32x4{0.f, 0.f, 0.f, 0.f});
                    c = mfma(al, bt[r].b[sb], c);
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[g][r][j] = fmaf(bt[r].dsc[sb], c[j], acc[g][r][j]);
                }
            }
#pragma unroll
            for (int r = 0; r < 2; r++) {
                f32x4 u = mfma(sx3[0], bt[r].bsc, f32x4{0.f, 0.f, 0.f, 0.f});
                u = mfma(sx3[1], bt[r].bsc, u);
                u = mfma(sx3[2], bt[r].bsc, u);
                const float cb = -(float)bias * bt[r].d;
#pragma unroll
                for (int j = 0; j < 4; j++) acc[g][r][j] = fmaf(cb, u[j], acc[g][r][j]);
                if (F != F_Q6K) {
                    f32x4 v = mfma(sx3[0], bt[r].bmin, f32x4{0.f, 0.f, 0.f, 0.f});
                    v = mfma(sx3[1], bt[r].bmin, v);
                    v = mfma(sx3[2], bt[r].bmin, v);
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[g][r][j] = fmaf(-bt[r].dmin, v[j], acc[g][r][j]);
                }
            }
        }
        __syncthreads();   // LDS is restaged for the next block
    }

    // epilogue: lane holds entries 16 g + 4 q + j of row n of its two tiles
#pragma unroll
    for (uint32_t g = 0; g < 2; g++) {
        if (g >= ngrp) break;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t m = 16 * g + 4 * q + j;
            if (m >= cnt) continue;
            const uint32_t e = ent0 + m;
            if (MODE == 0) {
                const float gv = acc[g][0][j], uv = acc[g][1][j];
                ws.mid[(size_t)e * L.inter + r0 + 16 * wave + n] = gv / (1.0f + expf(-gv)) * uv;
            } else {
                const float w = ws.ent_w[e];
                ws.ybuf[(size_t)e * L.hidden + r0 + 32 * wave + n] = w * acc[g][0][j];
                ws.ybuf[(size_t)e * L.hidden + r0 + 32 * wave + 16 + n] = w * acc[g][1][j];
            }
        }
    }
}

// out[t] = sum_k ybuf[entry(t, k)] + ybuf[shared entry(t)] (+ residual); the
// gate weights were applied by the down kernel. Selection order, shared last,
// as qw6.c:2263, 2284.
__global__ __launch_bounds__(256) void k_pre_combine(PrefillLayer L, PrefillWs ws) {
    const uint32_t t = blockIdx.x;
    uint32_t pos[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; k++) pos[k] = k < L.top_k ? ws.ent_pos[(size_t)t * L.top_k + k] : 0u;
    const bool sh = L.sg.p != nullptr;
    const uint32_t se = L.T * L.top_k + t;
    for (uint32_t i = threadIdx.x; i < L.hidden; i += blockDim.x) {
        float v = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < 8; k++)
            if (k < L.top_k) v += ws.ybuf[(size_t)pos[k] * L.hidden + i];
        if (sh) v += ws.ybuf[(size_t)se * L.hidden + i];
        if (L.residual) v += L.residual[(size_t)t * L.hidden + i];
        L.out[(size_t)t * L.hidden + i] = v;
    }
}

// y = rmsnorm(x) * w per token (qw6_cpu_rmsnorm, qw6.c:2503-2513).
__global__ __launch_bounds__(256) void k_pre_rmsnorm(const float* x, const float* w, float* y,
                                                     uint32_t n, float eps) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float sc = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 256) yr[i] = xr[i] * sc * w[i];
}

// Router logits of T tokens: block (expert e, tokens 4c .. 4c+3), one wave.
__global__ __launch_bounds__(64) void k_pre_router(const float* __restrict__ router,
                                                   const float* __restrict__ x, float* logits,
                                                   uint32_t n_experts, uint32_t hidden, uint32_t T) {
    const uint32_t e = blockIdx.x, t0 = 4 * blockIdx.y, lane = threadIdx.x;
    const float* wr = router + (size_t)e * hidden;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c = lane; c < hidden / 4; c += 64) {
        const float4 w = ((const float4*)wr)[c];
#pragma unroll
        for (uint32_t t = 0; t < 4; t++)
            if (t0 + t < T) {
                const float4 xv = ((const float4*)(x + (size_t)(t0 + t) * hidden))[c];
                acc[t] = fmaf(w.x, xv.x, acc[t]); acc[t] = fmaf(w.y, xv.y, acc[t]);
                acc[t] = fmaf(w.z, xv.z, acc[t]); acc[t] = fmaf(w.w, xv.w, acc[t]);
            }
    }
#pragma unroll
    for (uint32_t t = 0; t < 4; t++) {
        const float v = group_sum<64>(acc[t]);
        if (lane == 0 && t0 + t < T) logits[(size_t)(t0 + t) * n_experts + e] = v;
    }
}

template <int MODE>
int launch_gemm(int f, const PrefillLayer& L, const PrefillWs& ws, uint32_t grid_x,
                uint32_t grid_y, hipStream_t st) {
    const size_t lds = sizeof(GemmLds) - 4 + (size_t)kRaw * raw_chunks(f) * 16;
    switch (f) {
    case F_Q4K: k_pre_gemm<MODE, F_Q4K><<<dim3(grid_x, grid_y), kPWG, lds, st>>>(L, ws); break;
    case F_Q5K: k_pre_gemm<MODE, F_Q5K><<<dim3(grid_x, grid_y), kPWG, lds, st>>>(L, ws); break;
    case F_Q6K: k_pre_gemm<MODE, F_Q6K><<<dim3(grid_x, grid_y), kPWG, lds, st>>>(L, ws); break;
    default: return qw6_fail("batched path: unsupported weight format %d", f);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qw6_fail("batched kernel launch: %s", hipGetErrorString(e));
    return 0;
}

}  // namespace

uint32_t prefill_tiles_max(uint32_t T, uint32_t top_k, uint32_t n_experts) {
    return (T * top_k + kPM - 1) / kPM + n_experts + (T + kPM - 1) / kPM;
}

bool prefill_supports(int f) { return f == F_Q4K || f == F_Q5K || f == F_Q6K; }

int prefill_forward(const PrefillLayer& L, const PrefillWs& ws, hipStream_t st) {
    if (L.hidden % 256 || L.inter % 256 || L.inter % 64 || L.hidden % 128)
        return qw6_fail("batched path needs hidden, inter multiples of 256");
    if (!prefill_supports(L.fmt_gu) || !prefill_supports(L.fmt_dn))
        return qw6_fail("batched path: unsupported expert format");
    if (L.top_k == 0 || L.top_k > 8 || L.n_experts > 256)
        return qw6_fail("batched path: top_k / n_experts out of range");
    const float* xin = L.x;
    if (L.norm_w) {
        k_pre_rmsnorm<<<L.T, 256, 0, st>>>(L.x, L.norm_w, ws.xn, L.hidden, L.norm_eps);
        xin = ws.xn;
    }
    const float* logits = L.logits;
    if (!logits) {
        k_pre_router<<<dim3(L.n_experts, (L.T + 3) / 4), 64, 0, st>>>(L.router, xin, ws.logits,
                                                                    L.n_experts, L.hidden, L.T);
        logits = ws.logits;
    }
    PrefillLayer Lx = L;
    Lx.x = xin;
    k_pre_route<<<L.T, 64, 0, st>>>(Lx, ws, xin, logits);
    k_pre_sort<<<1, 1024, 0, st>>>(Lx, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qw6_fail("batched routing launch: %s", hipGetErrorString(e));
    const uint32_t nt = prefill_tiles_max(L.T, L.top_k, L.n_experts);
    if (launch_gemm<0>(L.fmt_gu, Lx, ws, nt, L.inter / 64, st)) return -1;
    if (launch_gemm<1>(L.fmt_dn, Lx, ws, nt, L.hidden / 128, st)) return -1;
    k_pre_combine<<<L.T, 256, 0, st>>>(Lx, ws);
    e = hipGetLastError();
    if (e != hipSuccess) return qw6_fail("batched combine launch: %s", hipGetErrorString(e));
    return 0;
}

}  // namespace qw6
