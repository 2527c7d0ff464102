// qw6_tile.h -- bf16 MFMA operands decoded from GGUF blocks staged in LDS,
// shared by the batched (qw6_prefill.hip) and small-batch (qw6_hip.hip)
// contractions on gfx950.
//
// Numerics: a weight enters the MFMA as its integer code, exact in bf16 (128 + q
// for a 4/5/6-bit code q: the byte pair {q, 0x43}; the signed lattice value for
// the IQ formats); the fp32 scales multiply the 16x16 results per sub-block, and
// the code bias and the K-quant minimum come back as (per-row integer) x
// (activation sum) products. Sub-blocks are 32 columns in every format here
// (Q6_K under qw6's even-scale rule, qw6.c:1567-1570).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw6_dev.h"

namespace qw6 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // register-resident 16 B

// 16-B chunks per staged row block: Q4_K / Q5_K blocks (144 / 176 B) of
// 16-byte aligned rows are 16-byte aligned; Q6_K (210 B) and IQ blocks (66,
// 82, 110 B) may start at any even offset within their first chunk.
__host__ __device__ constexpr uint32_t raw_chunks(int f) {
    return (f == F_Q4K || f == F_Q5K) ? fmt_block_bytes(f) / 16
                                      : (fmt_block_bytes(f) + 14 + 15) / 16;
}
__host__ __device__ constexpr bool is_iq(int f) {
    return f == F_IQ2XXS || f == F_IQ2S || f == F_IQ3S;
}
// LDS of the bf16 lattice grid of an IQ format (8 or 4 values per entry,
// 16 or 8 B); the signs are applied in registers (apply_signs).
__host__ __device__ constexpr uint32_t iq_grid_bytes(int f) {
    return f == F_IQ2XXS ? 256 * 16 : f == F_IQ2S ? 1024 * 16 : f == F_IQ3S ? 512 * 8 : 0;
}

// ---- bf16 operand preparation -----------------------------------------------------

__device__ __forceinline__ uint32_t bfb(__bf16 b) { return (uint32_t)__builtin_bit_cast(uint16_t, b); }

// A sub-block sum as three bf16 parts (hi, mid, lo), exact to fp32 precision.
__device__ __forceinline__ void split3(float x, uint16_t (&p)[3]) {
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const __bf16 b = (__bf16)x;
        p[i] = __builtin_bit_cast(uint16_t, b);
        x -= (float)b;
    }
}

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

// ---- B-tile decoding ----------------------------------------------------------------
// A tile is 16 weight rows. For one 256-column block, lane (n = l % 16,
// q = l / 16) reads row n's raw block bytes from LDS (s = LDS words, R = byte
// offset of the row's block) and produces, per sub-block s, the B operand:
// codes 128 + q (bf16) of columns 32 s + 8 q .. + 8.

// Per-tile scale state of one block: d * sc per sub-block, and d, dmin.
struct TileScales {
    float dsc[8];
    float d, dmin;
    uint32_t scw[2];   // the 8 sub-block scales as bytes (Q6_K: signed)
};

// The sub-block scales (and minimums) of row n as B operands over k =
// 8 q' + j (j = sub-block): lanes q' = 0, 1, 2 pair them with the three bf16
// parts of the activation sums; lanes q' = 3 meet a zero A operand.
// bf16 pair of two small integral floats (their low 16 bits are zero).
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

template <int F>
__device__ __forceinline__ void tile_scales(const uint32_t* s, uint32_t R, TileScales& ts,
                                            uint4& bsc, uint4& bmin) {
    float sc[8], mn[8];
    if (F == F_Q4K || F == F_Q5K) {
        const uint4 hd = *(const uint4*)(s + (R >> 2));   // 16-byte aligned block
        ts.d = h2f(hd.x & 0xffffu);
        ts.dmin = h2f(hd.x >> 16);
        // qw6_get_scale_min_k4 (qw6.c:1480-1490) for all eight sub-blocks at
        // once, four 6-bit values per word: j < 4 from the low 6 bits of bytes
        // 0-3 (scales) and 4-7 (minimums); j >= 4 from the nibbles of bytes
        // 8-11 with the top two bits of bytes j - 4 and j
        const uint32_t A = hd.y, B = hd.z, C = hd.w;
        const uint32_t sc_lo = A & 0x3f3f3f3fu, mn_lo = B & 0x3f3f3f3fu;
        const uint32_t sc_hi = (C & 0x0f0f0f0fu) | ((A >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((C >> 4) & 0x0f0f0f0fu) | ((B >> 2) & 0x30303030u);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sc[j] = ub(sc_lo, j);
            sc[j + 4] = ub(sc_hi, j);
            mn[j] = ub(mn_lo, j);
            mn[j + 4] = ub(mn_hi, j);
        }
        ts.scw[0] = sc_lo;
        ts.scw[1] = sc_hi;
    } else {   // Q6_K: sub-block 4h + k uses scale 8h + 2k (qw6.c:1550-1578)
        const LdsRow row = lds_row(R);
        ts.d = h2f(rd16(s, row, 208));
        ts.dmin = 0.f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t w0 = rd32(s, row, 192 + 8 * h), w1 = rd32(s, row, 196 + 8 * h);
            ts.scw[h] = __builtin_amdgcn_perm(w1, w0, 0x06040200u);   // bytes 0, 2 of w0, w1
            sc[4 * h + 0] = (float)(int8_t)(w0 & 0xffu);
            sc[4 * h + 1] = (float)(int8_t)((w0 >> 16) & 0xffu);
            sc[4 * h + 2] = (float)(int8_t)(w1 & 0xffu);
            sc[4 * h + 3] = (float)(int8_t)((w1 >> 16) & 0xffu);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) mn[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) ts.dsc[j] = ts.d * sc[j];
    bsc = u4(pk_bf16(sc[0], sc[1]), pk_bf16(sc[2], sc[3]), pk_bf16(sc[4], sc[5]), pk_bf16(sc[6], sc[7]));
    bmin = F != F_Q6K ? u4(pk_bf16(mn[0], mn[1]), pk_bf16(mn[2], mn[3]), pk_bf16(mn[4], mn[5]),
                           pk_bf16(mn[6], mn[7]))
                      : u4(0, 0, 0, 0);
}

// d * scale of sub-block sb from the packed bytes (the same value as
// ts.dsc[sb], computed where it is used instead of held in 8 registers).
template <int F>
__device__ __forceinline__ float tile_dsc(const TileScales& ts, int sb) {
    const uint32_t w = ts.scw[sb >> 2], sh = 8u * (uint32_t)(sb & 3);
    const float sc = F == F_Q6K ? (float)(int8_t)((w >> sh) & 0xffu) : (float)((w >> sh) & 0xffu);
    return ts.d * sc;
}

// Codes of sub-blocks 2p and 2p + 1 of row n (this lane's 8 columns of each).
template <int F>
__device__ __forceinline__ void tile_codes(const uint32_t* s, uint32_t R, uint32_t q, int p,
                                           uint4& b0, uint4& b1) {
    if (F == F_Q4K || F == F_Q5K) {
        // qs byte 32 p + l: low nibble column 64 p + l, high nibble 64 p + 32 + l
        const uint32_t qo = F == F_Q4K ? 16u : 48u;
        const uint2 wq = *(const uint2*)(s + ((R + qo + 32 * p + 8 * q) >> 2));
        uint32_t l0 = wq.x & 0x0f0f0f0fu, l1 = wq.y & 0x0f0f0f0fu;
        uint32_t h0 = (wq.x >> 4) & 0x0f0f0f0fu, h1 = (wq.y >> 4) & 0x0f0f0f0fu;
        if (F == F_Q5K) {   // qh byte l: bit 2p -> column 64 p + l, bit 2p + 1 -> + 32
            const uint2 hq = *(const uint2*)(s + ((R + 16 + 8 * q) >> 2));
            l0 |= ((hq.x >> (2 * p)) & 0x01010101u) << 4;
            l1 |= ((hq.y >> (2 * p)) & 0x01010101u) << 4;
            h0 |= ((hq.x >> (2 * p + 1)) & 0x01010101u) << 4;
            h1 |= ((hq.y >> (2 * p + 1)) & 0x01010101u) << 4;
        }
        b0 = codes8(l0, l1);
        b1 = codes8(h0, h1);
    } else {
        // half h = p / 2; sub-blocks 4h + 2i, 4h + 2i + 1 (i = p % 2): ql bytes
        // 64 h + l (a) and 64 h + 32 + l (b), low nibbles for i = 0, high for
        // i = 1; 2-bit fields 2k of qh byte 128 + 32 h + l (k = 2i, 2i + 1)
        const uint32_t h = (uint32_t)p >> 1, i = (uint32_t)p & 1u;
        const LdsRow rq = lds_row(R + 8 * q);
        const uint32_t a0 = rd32(s, rq, 64 * h), a1 = rd32(s, rq, 64 * h + 4);
        const uint32_t c0 = rd32(s, rq, 64 * h + 32), c1 = rd32(s, rq, 64 * h + 36);
        const uint32_t x0 = rd32(s, rq, 128 + 32 * h), x1 = rd32(s, rq, 132 + 32 * h);
        const uint32_t sh = 4 * i;   // nibble shift; also the qh shift 2k of k = 2i
        b0 = codes8(((a0 >> sh) & 0x0f0f0f0fu) | (((x0 >> sh) & 0x03030303u) << 4),
                    ((a1 >> sh) & 0x0f0f0f0fu) | (((x1 >> sh) & 0x03030303u) << 4));
        b1 = codes8(((c0 >> sh) & 0x0f0f0f0fu) | (((x0 >> (sh + 2)) & 0x03030303u) << 4),
                    ((c1 >> sh) & 0x0f0f0f0fu) | (((x1 >> (sh + 2)) & 0x03030303u) << 4));
    }
}

// ---- IQ formats -------------------------------------------------------------------
// The lattice values are small integers (IQ2: 8, 25, 43; IQ3: odd 1 .. 15),
// exact in bf16, and every weight is db * (+-value): the B operand is the
// bf16 grid entry with the sign bits flipped, with no bias or minimum term.

// Expand the lattice grid of format F into LDS as bf16 at `grid` (8 or 4
// values per entry, 16 or 8 B). All nthr threads of the workgroup take part;
// g: the lattice tables.
template <int F>
__device__ __forceinline__ void stage_iq_grid(uint8_t* grid, const IqTables& g, uint32_t nthr) {
    const uint32_t tid = threadIdx.x;
    auto bf = [](uint32_t v) { return bf16_bits((float)v); };
    if (F == F_IQ2XXS || F == F_IQ2S) {
        const uint32_t n = F == F_IQ2XXS ? 256u : 1024u;
        const uint64_t* src = F == F_IQ2XXS ? g.iq2xxs : g.iq2s;
        for (uint32_t i = tid; i < n; i += nthr) {
            const uint64_t v = src[i];
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                w[k] = bf((uint32_t)(v >> (16 * k)) & 255u) | (bf((uint32_t)(v >> (16 * k + 8)) & 255u) << 16);
            ((uint4*)grid)[i] = u4(w[0], w[1], w[2], w[3]);
        }
    } else if (F == F_IQ3S) {
        for (uint32_t i = tid; i < 512; i += nthr) {
            const uint32_t v = g.iq3s[i];
            ((uint2*)grid)[i] = make_uint2(bf(v & 255u) | (bf((v >> 8) & 255u) << 16),
                                           bf((v >> 16) & 255u) | (bf(v >> 24) << 16));
        }
    }
}

// Signs of 8 bf16 values g (value h: 16-bit half h of g) from bits 0-7 of
// both 16-bit halves of y (bit h -> value h): the halves of word k shift by
// 15 - 2k and 14 - 2k (one packed 16-bit shift), which puts bit 2k, 2k + 1
// on bits 15, 31; bits that leave a half are dropped and the rest masked off.
// Bits 8-15 of a half shift out for every k, so they may hold anything.
typedef unsigned short us2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 apply_signs(const uint4& g, uint32_t y) {
    const us2_t v = __builtin_bit_cast(us2_t, y);
    uint32_t m[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const us2_t sh = {(unsigned short)(15 - 2 * k), (unsigned short)(14 - 2 * k)};
        m[k] = __builtin_bit_cast(uint32_t, (us2_t)(v << sh)) & 0x80008000u;
    }
    return u4(g.x ^ m[0], g.y ^ m[1], g.z ^ m[2], g.w ^ m[3]);
}
// y for apply_signs from a sign byte s8 (bits 8+ of s8 may be set), and from
// IQ2_XXS's 7 stored bits s7, whose eighth is their parity (ksigns_iq2xs):
// the popcount lands on bits 23-25, its low bit on bit 7 of the high half;
// the low half's bit 7 goes to no value (even values take bits 0, 2, 4, 6).
__device__ __forceinline__ uint32_t sign_pairs(uint32_t s8) { return s8 | (s8 << 16); }
__device__ __forceinline__ uint32_t sign_pairs7(uint32_t s7) {
    return s7 | (s7 << 16) | ((uint32_t)__builtin_popcount(s7) << 23);
}

// B operand of sub-block sb of row n (this lane's 8 weights, group q of the
// sub-block; tab: the bf16 grid) and its scale(s): db for all 32 weights, or
// (IQ2_S) db for groups 0-1 and db2 for groups 2-3 (qw6.c:1580-1672).
template <int F>
__device__ __forceinline__ void tile_iq(const uint32_t* s, const uint8_t* tab,
                                        uint32_t R, uint32_t q, int sb, float d, uint4& b,
                                        float& db, float& db2) {
    const LdsRow row = lds_row(R);
    if (F == F_IQ2XXS) {   // 8 B per 32 weights: 4 grid indices, 4 x 7 sign bits + scale
        const uint32_t aux0 = rd32(s, row, 2 + 8 * sb), aux1 = rd32(s, row, 6 + 8 * sb);
        const uint32_t idx = (aux0 >> (8 * q)) & 255u;
        const uint32_t s7 = (aux1 >> (7 * q)) & 127u;
        b = apply_signs(((const uint4*)tab)[idx], sign_pairs7(s7));
        db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
        db2 = db;
    } else if (F == F_IQ2S) {   // grid index: qs byte + 2 bits of qh; own sign byte
        const uint32_t qsb = (rd32(s, row, 2 + 4 * sb) >> (8 * q)) & 0xffu;
        const uint32_t qh = rd8(s, row, 66 + sb);
        const uint32_t sg = (rd32(s, row, 34 + 4 * sb) >> (8 * q)) & 0xffu;
        const uint32_t sc = rd8(s, row, 74 + sb);
        const uint32_t gi = qsb | ((qh << (8 - 2 * q)) & 0x300u);
        b = apply_signs(((const uint4*)tab)[gi], sign_pairs(sg));
        db = d * (0.5f + (float)(sc & 15u)) * 0.25f;
        db2 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
    } else {   // IQ3_S: two 4-value grid entries per 8 weights, 9-bit indices
        const LdsRow rq = lds_row(R + 4 * (q >> 1));
        const uint32_t qw = rd32(s, rq, 2 + 8 * sb);
        const uint32_t qh = rd8(s, row, 66 + sb);
        const uint32_t sg = (rd32(s, row, 74 + 4 * sb) >> (8 * q)) & 0xffu;
        const uint32_t scb = rd8(s, row, 106 + (sb >> 1));
        const uint32_t nib = (sb & 1) ? (scb >> 4) : (scb & 15u);
        const uint32_t sh = 16 * (q & 1u);
        const uint32_t i1 = ((qw >> sh) & 255u) | ((qh << (8 - 2 * q)) & 256u);
        const uint32_t i2 = ((qw >> (sh + 8)) & 255u) | ((qh << (7 - 2 * q)) & 256u);
        const uint2 g1 = ((const uint2*)tab)[i1], g2 = ((const uint2*)tab)[i2];
        b = apply_signs(u4(g1.x, g1.y, g2.x, g2.y), sign_pairs(sg));
        db = d * (float)(1 + 2 * (int)nib);
        db2 = db;
    }
}

// ---- small-batch block product ------------------------------------------------------
// One 256-column block of a 16-row weight tile (lane: row n = l % 16 at LDS
// byte offset R, k group q = l / 16) against token-row A operands: a[j] for
// sub-block j, c0 / c1 the bias / minimum operands over the two halves of the
// sub-blocks (3-part half-sums in k-slots 8 part + j, zero elsewhere).
// acc += the block's contribution to D[m][n], this lane's rows m = 4 q + i.
template <int F>
__device__ __forceinline__ void mx_block(const uint32_t* s, const uint8_t* grid,
                                         uint32_t R, uint32_t q, const uint4 (&a)[8],
                                         const uint4& c0, const uint4& c1, f32x4& acc) {
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (is_iq(F)) {
        const float d = h2f(rd16(s, lds_row(R), 0));
#pragma unroll
        for (int sb = 0; sb < 8; sb++) {
            uint4 b;
            float db, db2;
            tile_iq<F>(s, grid, R, q, sb, d, b, db, db2);
            if (F == F_IQ2S) {   // scales per 16 weights: groups 0-1, then 2-3
                const uint4 z = u4(0, 0, 0, 0);
                const f32x4 c = mfma(a[sb], q < 2 ? b : z, z4);
                const f32x4 c1v = mfma(a[sb], q < 2 ? z : b, z4);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = fmaf(db2, c1v[i], fmaf(db, c[i], acc[i]));
            } else {
                const f32x4 c = mfma(a[sb], b, z4);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = fmaf(db, c[i], acc[i]);
            }
            if (sb & 1) __builtin_amdgcn_sched_barrier(0);   // two sub-blocks' operands live at a time
        }
        return;
    }
    constexpr float bias = F == F_Q6K ? 160.f : 128.f;
    TileScales ts;
    uint4 bsc, bmin;
    tile_scales<F>(s, R, ts, bsc, bmin);
    const f32x4 u = mfma(c1, bsc, mfma(c0, bsc, z4));
    const float cb = -bias * ts.d;
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = fmaf(cb, u[i], acc[i]);
    if (F != F_Q6K) {
        const f32x4 v = mfma(c1, bmin, mfma(c0, bmin, z4));
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(-ts.dmin, v[i], acc[i]);
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        uint4 b0, b1;
        tile_codes<F>(s, R, q, p, b0, b1);
        const f32x4 e0 = mfma(a[2 * p], b0, z4);
        const f32x4 e1 = mfma(a[2 * p + 1], b1, z4);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(ts.dsc[2 * p + 1], e1[i], fmaf(ts.dsc[2 * p], e0[i], acc[i]));
        __builtin_amdgcn_sched_barrier(0);   // one sub-block pair's operands live at a time
    }
}

}  // namespace qw6
