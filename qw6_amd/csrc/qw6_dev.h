// qw6_dev.h -- device building blocks of the gfx950 MoE FFN kernels.
//
// GGUF super-block decoders that turn one 32-weight "unit" of a block into a
// dot product with activations held in registers, the IQ lattice tables as
// device constants (staged into LDS by the kernels that need them), exact
// fp16 decoding, LDS byte readers for blocks that are only 2-byte aligned,
// and wave64 reductions.
//
// Unit j (0..7) of a 256-weight block covers 32 columns of that block:
//   Q4_K / Q5_K: qs bytes [16j, 16j+16): low nibbles are columns
//                64(j/2) + 16(j%2) + i, high nibbles the same + 32 (i < 16);
//   Q6_K:        half h = j/4, l in [8(j%4), 8(j%4)+8): columns
//                128h + 32k + l for k = 0..3;
//   IQ2_XXS / IQ2_S / IQ3_S: columns 32j .. 32j+31.
// Each unit only needs its own bytes plus the block header, so a lane can
// keep the same unit across rows with its 32 activations in registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq_grid_data.h"

namespace qw6 {

enum Fmt : int { F_Q4K = 0, F_Q5K = 1, F_Q6K = 2, F_IQ2XXS = 3, F_IQ2S = 4, F_IQ3S = 5, F_NFMT = 6 };

// qw6_quant_t (qw6.h:76-91) -> internal format, -1 if no block decoder.
__host__ __device__ inline int fmt_of_quant(int q) {
    switch (q) {
    case 4: case 5: return F_Q4K;
    case 6: return F_Q5K;
    case 7: return F_Q6K;
    case 13: return F_IQ2XXS;
    case 11: return F_IQ2S;
    case 9: return F_IQ3S;
    default: return -1;
    }
}

__host__ __device__ constexpr uint32_t fmt_block_bytes(int f) {
    switch (f) {
    case F_Q4K: return 144;
    case F_Q5K: return 176;
    case F_Q6K: return 210;
    case F_IQ2XXS: return 66;
    case F_IQ2S: return 82;
    default: return 110;
    }
}

// Which LDS lattice tables a format needs (bit 0: iq2xxs, 1: iq2s, 2: iq3s).
__host__ __device__ inline uint32_t fmt_table_mask(int f) {
    return f == F_IQ2XXS ? 1u : f == F_IQ2S ? 2u : f == F_IQ3S ? 4u : 0u;
}

// ---- IQ lattice tables --------------------------------------------------------

// Per-token decoders read the tables from LDS at these offsets. Besides the
// lattice grids they hold byte sign masks: entry s has byte n = 0xff when
// weight n of the group of 8 is negative, else 0 (sgnxx is indexed by the
// 7-bit IQ2_XXS sign field, whose eighth sign makes the count of negative
// signs even, qw6.c:1590-1596; sgn8 by a plain sign byte). With them a
// group's 8 signed grid values come from two integer ops per 4 bytes.
struct IqTables {
    uint64_t sgnxx[128];
    uint64_t iq2xxs[256];
    uint64_t sgn8[256];
    uint32_t iq3s[512];
    uint64_t iq2s[1024];
};
constexpr uint32_t kTabOffSgnXX = 0;
constexpr uint32_t kTabOffIq2xxs = 128 * 8;
constexpr uint32_t kTabOffSgn8 = kTabOffIq2xxs + 256 * 8;
constexpr uint32_t kTabOffIq3s = kTabOffSgn8 + 256 * 8;
constexpr uint32_t kTabOffIq2s = kTabOffIq3s + 512 * 4;
constexpr uint32_t kTabBytes = kTabOffIq2s + 1024 * 8;   // 15 KB

constexpr uint64_t expand_iq2(uint16_t c) {
    uint64_t v = 0;
    for (int j = 0; j < 8; j++) v |= (uint64_t)QW6_IQ2_LEVEL((c >> (2 * j)) & 3) << (8 * j);
    return v;
}
constexpr uint32_t expand_iq3(uint16_t c) {
    uint32_t v = 0;
    for (int j = 0; j < 4; j++) v |= (uint32_t)(2 * ((c >> (3 * j)) & 7) + 1) << (8 * j);
    return v;
}
constexpr uint64_t sign_mask8(uint32_t s) {
    uint64_t v = 0;
    for (int n = 0; n < 8; n++)
        if ((s >> n) & 1u) v |= (uint64_t)0xffu << (8 * n);
    return v;
}
constexpr uint32_t parity7(uint32_t s) {
    uint32_t p = 0;
    for (int n = 0; n < 7; n++) p ^= (s >> n) & 1u;
    return p;
}
constexpr IqTables make_tables() {
    IqTables t{};
    for (uint32_t i = 0; i < 128; i++) t.sgnxx[i] = sign_mask8(i | (parity7(i) << 7));
    for (uint32_t i = 0; i < 256; i++) t.sgn8[i] = sign_mask8(i);
    for (int i = 0; i < 256; i++) t.iq2xxs[i] = expand_iq2(qw6_iq2xxs_codes[i]);
    for (int i = 0; i < 1024; i++) t.iq2s[i] = expand_iq2(qw6_iq2s_codes[i]);
    for (int i = 0; i < 512; i++) t.iq3s[i] = expand_iq3(qw6_iq3s_codes[i]);
    return t;
}
static_assert(__builtin_offsetof(IqTables, iq2xxs) == kTabOffIq2xxs &&
              __builtin_offsetof(IqTables, sgn8) == kTabOffSgn8 &&
              __builtin_offsetof(IqTables, iq3s) == kTabOffIq3s &&
              __builtin_offsetof(IqTables, iq2s) == kTabOffIq2s && sizeof(IqTables) == kTabBytes,
              "LDS table offsets");

// ---- scalar helpers ------------------------------------------------------------

// Exact binary16 -> binary32: v_cvt_f32_f16. The kernels run with f16 and
// f32 denormals preserved (denorm mode 3 in every kernel descriptor), so
// subnormal halves convert to their exact normal f32 values (qw6.c:1448-1471).
__device__ __forceinline__ float h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// float -> binary16, round to nearest even, subnormals kept (synthetic data).
__host__ __device__ inline uint16_t f2h_rne(float f) {
    uint32_t x;
    __builtin_memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   // rounds to inf
    const int e = (int)(ax >> 23) - 127;
    if (e < -25) return (uint16_t)sign;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    int shift;                   // bits dropped from the 24-bit significand
    uint32_t base;
    if (e < -14) { shift = 13 + (-14 - e); base = 0; }
    else { shift = 13; base = (uint32_t)(e + 15) << 10; mant &= 0x7fffffu; }
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | (base + q));   // carry into the exponent is correct
}

// ---- LDS byte readers ---------------------------------------------------------
// s: LDS viewed as 32-bit words; off: byte offset.

__device__ __forceinline__ uint32_t lds8(const uint32_t* s, uint32_t off) {
    return (s[off >> 2] >> ((off & 3) * 8)) & 0xffu;
}
// Reads at R + c from an even LDS byte offset R (every staged block starts at
// an even byte) with c a constant after inlining: R is kept as the word
// indices and byte shifts of R and R + 2, so a read needs no address
// arithmetic (the word is w0 + c / 4 or w2 + (c - 2) / 4, a ds_read offset)
// and a dword one v_alignbyte. Build the cursor once per block with lds_row.
struct LdsRow {
    uint32_t w0, w2;   // (R >> 2), ((R + 2) >> 2)
    uint32_t s0, s2;   // R & 3, (R + 2) & 3 (bytes: 0 or 2)
};
__device__ __forceinline__ LdsRow lds_row(uint32_t R) {
    return LdsRow{R >> 2, (R + 2u) >> 2, R & 3u, (R + 2u) & 3u};
}
__device__ __forceinline__ uint32_t row_word(const LdsRow& r, uint32_t c) {   // c even
    return (c & 2u) ? r.w2 + ((c - 2u) >> 2) : r.w0 + (c >> 2);
}
__device__ __forceinline__ uint32_t row_shift(const LdsRow& r, uint32_t c) {   // bytes
    return ((c & 2u) ? r.s2 : r.s0) + (c & 1u);
}
__device__ __forceinline__ uint32_t rd32(const uint32_t* s, const LdsRow& r, uint32_t c) {   // c even
    const uint32_t w = row_word(r, c);
    return __builtin_amdgcn_alignbyte(s[w + 1], s[w], row_shift(r, c));
}
__device__ __forceinline__ uint32_t rd16(const uint32_t* s, const LdsRow& r, uint32_t c) {   // c even
    return (s[row_word(r, c)] >> (8u * row_shift(r, c))) & 0xffffu;
}
__device__ __forceinline__ uint32_t rd8(const uint32_t* s, const LdsRow& r, uint32_t c) {
    return (s[row_word(r, c & ~1u)] >> (8u * row_shift(r, c))) & 0xffu;
}

__device__ __forceinline__ uint64_t lds64_tab(const uint32_t* s, uint32_t off) {
    const uint2 v = *(const uint2*)(s + (off >> 2));   // 8-byte aligned table entry
    return (uint64_t)v.x | ((uint64_t)v.y << 32);
}

// Byte n of w as a float: one v_cvt_f32_ubyteN (the compiler would otherwise
// emit a bit-field extract plus a conversion).
__device__ __forceinline__ float ub(uint32_t w, int n) {
    float r;
    switch (n) {
    case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w)); break;
    case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w)); break;
    case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w)); break;
    default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w)); break;
    }
    return r;
}
// Four grid bytes g (each 1..63) with the signs of byte mask m (0xff =
// negative) as int8: (g ^ 0xff) + 1 = 256 - g per negated byte, no carry
// between bytes since g > 0 (v_and + v_xad_u32).
__device__ __forceinline__ uint32_t signed_bytes(uint32_t g, uint32_t m) {
    uint32_t r;
    asm("v_xad_u32 %0, %1, %2, %3" : "=v"(r) : "v"(g), "v"(m), "v"(m & 0x01010101u));
    return r;
}
// Signed byte n of w as a float: one v_cvt_f32_i32 with a sign-extending
// byte source select.
__device__ __forceinline__ float sb(uint32_t w, int n) { return (float)(int8_t)(w >> (8 * n)); }

// ---- activations for a unit ------------------------------------------------------

// Activation layout class of a format's units (load_unit_x): Q4_K and Q5_K
// share one, Q6_K has its own, the IQ formats read 32 contiguous values.
__host__ __device__ inline int x_layout(int f) {
    return (f == F_Q4K || f == F_Q5K) ? 0 : f == F_Q6K ? 1 : 2;
}

// Load the 32 activations of unit j of block blk for format f from x (one
// token, contiguous). The partial sums the K-quant decoders use come from
// unit_x_sums, separately, so that a caller can issue further loads before
// it waits for these.
__device__ __forceinline__ void load_unit_x(int f, const float* __restrict__ x, uint32_t blk,
                                            int j, float (&xr)[32]) {
    // Load i fills xr[4i .. 4i+3] in every layout; only the addresses differ:
    // Q4_K/Q5_K the runs 64(j/2) + 16(j%2) and +32 (16 values each), Q6_K
    // the 8-runs 128(j/4) + 8(j%4) + 32k, IQ 32 contiguous values at 32j. The
    // offsets are selected, not branched on, so a run-time format leaves one
    // straight load sequence (no merge of alternative loads into the same
    // registers, which would make the compiler wait for them).
    const int lay = x_layout(f);
    const uint32_t ju = (uint32_t)j;
    const uint32_t base = lay == 0 ? 64u * (ju >> 1) + 16u * (ju & 1)
                        : lay == 1 ? 128u * (ju >> 2) + 8u * (ju & 3) : 32u * ju;
    const float* b = x + blk * 256 + base;
#pragma unroll
    for (uint32_t i = 0; i < 8; i++) {
        const uint32_t add = lay == 0 ? 4u * i + (i >= 4 ? 16u : 0u)
                           : lay == 1 ? 32u * (i >> 1) + 4u * (i & 1) : 4u * i;
        const float4 v = *(const float4*)(b + add);
        xr[4 * i] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
    }
}

// Partial activation sums of a unit for format f (Q4_K/Q5_K: the two 16-runs;
// Q6_K: the four 8-runs; the IQ decoders use none).
__device__ __forceinline__ void unit_x_sums(int f, const float (&xr)[32], float (&sx)[4]) {
    if (f == F_Q6K) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) s += xr[8 * k + i];
            sx[k] = s;
        }
    } else if (f == F_Q4K || f == F_Q5K) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) { s0 += xr[i]; s1 += xr[16 + i]; }
        sx[0] = s0; sx[1] = s1; sx[2] = 0.f; sx[3] = 0.f;
    } else {   // the IQ decoders use no activation sums
        sx[0] = sx[1] = sx[2] = sx[3] = 0.f;
    }
}

// ---- unit decoders: acc[t] += sum_i w_i * xr[t][i] ----------------------------
// s: LDS words; bo: byte offset of the block in LDS; tab: LDS words of the
// lattice tables (IqTables layout at offset 0).

// Q4_K / Q5_K block scales (qw6_get_scale_min_k4, qw6.c:1480-1490). The 8
// lanes of a block hold units j = 0..7 (lane & 7); lane j decodes sub-block
// j's 6-bit (scale, min) and two quad permutes hand every lane the pair of
// its own unit, sub-blocks 2(j/2) (low nibbles) and 2(j/2)+1 (high nibbles).
// hdr = the block's first 16 bytes {d|dmin, scales[0..3], [4..7], [8..11]}.
struct KScales {
    float da, ma, db, mb;   // d*sc and dmin*m of the low / high sub-block
};
__device__ __forceinline__ KScales k_scales(const uint4& hdr, int j) {
    const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const uint32_t sc_lo = __builtin_amdgcn_ubfe(hdr.y, sh, 6);
    const uint32_t m_lo = __builtin_amdgcn_ubfe(hdr.z, sh, 6);
    const uint32_t sc_hi = __builtin_amdgcn_ubfe(hdr.w, sh, 4) | (__builtin_amdgcn_ubfe(hdr.y, sh + 6, 2) << 4);
    const uint32_t m_hi = __builtin_amdgcn_ubfe(hdr.w, sh + 4, 4) | (__builtin_amdgcn_ubfe(hdr.z, sh + 6, 2) << 4);
    const float fd = d * (float)(j < 4 ? sc_lo : sc_hi);
    const float fm = dmin * (float)(j < 4 ? m_lo : m_hi);
    const uint32_t ud = __float_as_uint(fd), um = __float_as_uint(fm);
    KScales k;
    k.da = __uint_as_float(__builtin_amdgcn_update_dpp(0u, ud, 0xA0, 0xf, 0xf, false));  // [0,0,2,2]
    k.db = __uint_as_float(__builtin_amdgcn_update_dpp(0u, ud, 0xF5, 0xf, 0xf, false));  // [1,1,3,3]
    k.ma = __uint_as_float(__builtin_amdgcn_update_dpp(0u, um, 0xA0, 0xf, 0xf, false));
    k.mb = __uint_as_float(__builtin_amdgcn_update_dpp(0u, um, 0xF5, 0xf, 0xf, false));
    return k;
}

// Q4_K (qw6.c:1492-1516): w = (d*sc)*q - dmin*m per 32-run. Blocks are 144 B,
// so bo is 16-byte aligned.
template <int T>
__device__ __forceinline__ void unit_q4k(const uint32_t* s, uint32_t bo, int j,
                                         const float (&xr)[T][32], const float (&sx)[T][4],
                                         float (&acc)[T]) {
    const uint4 hdr = *(const uint4*)(s + (bo >> 2));
    const uint4 q = *(const uint4*)(s + ((bo + 16 + 16 * j) >> 2));
    const KScales k = k_scales(hdr, j);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    float lo[T], hi[T];
#pragma unroll
    for (int t = 0; t < T; t++) { lo[t] = 0.f; hi[t] = 0.f; }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t l4 = qw[i] & 0x0f0f0f0fu, h4 = (qw[i] >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const float fl = ub(l4, n), fh = ub(h4, n);
#pragma unroll
            for (int t = 0; t < T; t++) {
                lo[t] = fmaf(fl, xr[t][4 * i + n], lo[t]);
                hi[t] = fmaf(fh, xr[t][16 + 4 * i + n], hi[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++)
        acc[t] += (k.da * lo[t] - k.ma * sx[t][0]) + (k.db * hi[t] - k.mb * sx[t][1]);
}

// Q5_K (qw6.c:1518-1548): as Q4_K with a fifth bit from qh. Blocks are 176 B.
template <int T>
__device__ __forceinline__ void unit_q5k(const uint32_t* s, uint32_t bo, int j,
                                         const float (&xr)[T][32], const float (&sx)[T][4],
                                         float (&acc)[T]) {
    const uint4 hdr = *(const uint4*)(s + (bo >> 2));
    const uint4 q = *(const uint4*)(s + ((bo + 48 + 16 * j) >> 2));
    const uint4 h = *(const uint4*)(s + ((bo + 16 + 16 * (j & 1)) >> 2));
    const KScales k = k_scales(hdr, j);
    const uint32_t sa = 2u * (uint32_t)(j >> 1), sb = sa + 1;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
    float lo[T], hi[T];
#pragma unroll
    for (int t = 0; t < T; t++) { lo[t] = 0.f; hi[t] = 0.f; }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t l5 = (qw[i] & 0x0f0f0f0fu) | (((hw[i] >> sa) & 0x01010101u) << 4);
        const uint32_t h5 = ((qw[i] >> 4) & 0x0f0f0f0fu) | (((hw[i] >> sb) & 0x01010101u) << 4);
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const float fl = ub(l5, n), fh = ub(h5, n);
#pragma unroll
            for (int t = 0; t < T; t++) {
                lo[t] = fmaf(fl, xr[t][4 * i + n], lo[t]);
                hi[t] = fmaf(fh, xr[t][16 + 4 * i + n], hi[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++)
        acc[t] += (k.da * lo[t] - k.ma * sx[t][0]) + (k.db * hi[t] - k.mb * sx[t][1]);
}

// Q6_K (qw6.c:1550-1578), qw6's even-scale rule: the 32-run k of half h uses
// scales[8h + 2k] for all its weights.
template <int T>
__device__ __forceinline__ void unit_q6k(const uint32_t* s, uint32_t bo, int j,
                                         const float (&xr)[T][32], const float (&sx)[T][4],
                                         float (&acc)[T]) {
    const int h = j >> 2, lq = j & 3;
    const LdsRow ra = lds_row(bo + 64 * h + 8 * lq), rh = lds_row(bo + 128 + 32 * h + 8 * lq);
    const LdsRow rs = lds_row(bo + 8 * h), rb = lds_row(bo);
    const uint32_t a0 = rd32(s, ra, 0), a1 = rd32(s, ra, 4);
    const uint32_t b0 = rd32(s, ra, 32), b1 = rd32(s, ra, 36);
    const uint32_t h0 = rd32(s, rh, 0), h1 = rd32(s, rh, 4);
    const uint32_t sc0 = rd32(s, rs, 192), sc1 = rd32(s, rs, 196);
    const float d = h2f(rd16(s, rb, 208));
    const float sc[4] = {(float)(int8_t)(sc0 & 0xff), (float)(int8_t)((sc0 >> 16) & 0xff),
                         (float)(int8_t)(sc1 & 0xff), (float)(int8_t)((sc1 >> 16) & 0xff)};
    const uint32_t aw[2] = {a0, a1}, bw[2] = {b0, b1}, hw[2] = {h0, h1};
    float part[T][4];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int k = 0; k < 4; k++) part[t][k] = 0.f;
#pragma unroll
    for (int w = 0; w < 2; w++) {
        const uint32_t v0 = (aw[w] & 0x0f0f0f0fu) | ((hw[w] & 0x03030303u) << 4);
        const uint32_t v1 = (bw[w] & 0x0f0f0f0fu) | (((hw[w] >> 2) & 0x03030303u) << 4);
        const uint32_t v2 = ((aw[w] >> 4) & 0x0f0f0f0fu) | (((hw[w] >> 4) & 0x03030303u) << 4);
        const uint32_t v3 = ((bw[w] >> 4) & 0x0f0f0f0fu) | (((hw[w] >> 6) & 0x03030303u) << 4);
        const uint32_t vv[4] = {v0, v1, v2, v3};
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int n = 0; n < 4; n++) {
                const float fv = ub(vv[k], n);
#pragma unroll
                for (int t = 0; t < T; t++)
                    part[t][k] = fmaf(fv, xr[t][8 * k + 4 * w + n], part[t][k]);
            }
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        float r = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) r += (d * sc[k]) * (part[t][k] - 32.f * sx[t][k]);
        acc[t] += r;
    }
}

// IQ2_XXS (qw6.c:1580-1602).
template <int T>
__device__ __forceinline__ void unit_iq2xxs(const uint32_t* s, uint32_t bo, int j,
                                            const uint32_t* tab, const float (&xr)[T][32],
                                            float (&acc)[T]) {
    const LdsRow rj = lds_row(bo + 8 * j);
    const uint32_t aux0 = rd32(s, rj, 2), aux1 = rd32(s, rj, 6);
    const float d = h2f(rd16(s, lds_row(bo), 0));
    const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
    float sum[T];
#pragma unroll
    for (int t = 0; t < T; t++) sum[t] = 0.f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint64_t g = lds64_tab(tab, kTabOffIq2xxs + 8 * ((aux0 >> (8 * l)) & 0xffu));
        const uint64_t m = lds64_tab(tab, kTabOffSgnXX + 8 * ((aux1 >> (7 * l)) & 127u));
        const uint32_t w0 = signed_bytes((uint32_t)g, (uint32_t)m);
        const uint32_t w1 = signed_bytes((uint32_t)(g >> 32), (uint32_t)(m >> 32));
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const float gv = sb(n < 4 ? w0 : w1, n & 3);
#pragma unroll
            for (int t = 0; t < T; t++) sum[t] = fmaf(gv, xr[t][8 * l + n], sum[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] += db * sum[t];
}

// IQ2_S (qw6.c:1604-1630).
template <int T>
__device__ __forceinline__ void unit_iq2s(const uint32_t* s, uint32_t bo, int j,
                                          const uint32_t* tab, const float (&xr)[T][32],
                                          float (&acc)[T]) {
    const LdsRow rj = lds_row(bo + 4 * j), rb = lds_row(bo);
    const uint32_t qs4 = rd32(s, rj, 2), sg4 = rd32(s, rj, 34);
    const uint32_t qh = lds8(s, bo + 66 + j), sc = lds8(s, bo + 74 + j);
    const float d = h2f(rd16(s, rb, 0));
    const float db0 = d * (0.5f + (float)(sc & 0xf)) * 0.25f;
    const float db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
    float s0[T], s1[T];
#pragma unroll
    for (int t = 0; t < T; t++) { s0[t] = 0.f; s1[t] = 0.f; }
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint32_t gi = ((qs4 >> (8 * l)) & 0xffu) | ((qh << (8 - 2 * l)) & 0x300u);
        const uint64_t g = lds64_tab(tab, kTabOffIq2s + 8 * gi);
        const uint64_t m = lds64_tab(tab, kTabOffSgn8 + 8 * ((sg4 >> (8 * l)) & 0xffu));
        const uint32_t w0 = signed_bytes((uint32_t)g, (uint32_t)m);
        const uint32_t w1 = signed_bytes((uint32_t)(g >> 32), (uint32_t)(m >> 32));
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const float gv = sb(n < 4 ? w0 : w1, n & 3);
#pragma unroll
            for (int t = 0; t < T; t++) {
                if (l < 2) s0[t] = fmaf(gv, xr[t][8 * l + n], s0[t]);
                else s1[t] = fmaf(gv, xr[t][8 * l + n], s1[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] += db0 * s0[t] + db1 * s1[t];
}

// IQ3_S (qw6.c:1632-1672).
template <int T>
__device__ __forceinline__ void unit_iq3s(const uint32_t* s, uint32_t bo, int j,
                                          const uint32_t* tab, const float (&xr)[T][32],
                                          float (&acc)[T]) {
    const LdsRow r8 = lds_row(bo + 8 * j), r4 = lds_row(bo + 4 * j);
    const uint32_t qa = rd32(s, r8, 2), qb = rd32(s, r8, 6);
    const uint32_t qh = lds8(s, bo + 66 + j);
    const uint32_t sg4 = rd32(s, r4, 74);
    const uint32_t scb = lds8(s, bo + 106 + (j >> 1));
    const uint32_t nib = (j & 1) ? (scb >> 4) : (scb & 0xf);
    const float d = h2f(rd16(s, lds_row(bo), 0));
    const float db = d * (float)(1 + 2 * (int)nib);
    float sum[T];
#pragma unroll
    for (int t = 0; t < T; t++) sum[t] = 0.f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint32_t qw = l < 2 ? qa : qb;
        const uint32_t i1 = ((qw >> (16 * (l & 1))) & 0xffu) | ((qh << (8 - 2 * l)) & 256u);
        const uint32_t i2 = ((qw >> (16 * (l & 1) + 8)) & 0xffu) | ((qh << (7 - 2 * l)) & 256u);
        const uint64_t m = lds64_tab(tab, kTabOffSgn8 + 8 * ((sg4 >> (8 * l)) & 0xffu));
        const uint32_t w1 = signed_bytes(tab[(kTabOffIq3s >> 2) + i1], (uint32_t)m);
        const uint32_t w2 = signed_bytes(tab[(kTabOffIq3s >> 2) + i2], (uint32_t)(m >> 32));
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const float v1 = sb(w1, n), v2 = sb(w2, n);
#pragma unroll
            for (int t = 0; t < T; t++) {
                sum[t] = fmaf(v1, xr[t][8 * l + n], sum[t]);
                sum[t] = fmaf(v2, xr[t][8 * l + 4 + n], sum[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] += db * sum[t];
}

template <int T>
__device__ __forceinline__ void unit_dot(int f, const uint32_t* s, uint32_t bo, int j,
                                         const uint32_t* tab, const float (&xr)[T][32],
                                         const float (&sx)[T][4], float (&acc)[T]) {
    switch (f) {
    case F_Q4K: unit_q4k<T>(s, bo, j, xr, sx, acc); break;
    case F_Q5K: unit_q5k<T>(s, bo, j, xr, sx, acc); break;
    case F_Q6K: unit_q6k<T>(s, bo, j, xr, sx, acc); break;
    case F_IQ2XXS: unit_iq2xxs<T>(s, bo, j, tab, xr, acc); break;
    case F_IQ2S: unit_iq2s<T>(s, bo, j, tab, xr, acc); break;
    default: unit_iq3s<T>(s, bo, j, tab, xr, acc); break;
    }
}

// ---- reductions ----------------------------------------------------------------
// Lane exchanges at distance m within aligned groups, without LDS traffic:
// m = 32 / 16 swap halves / odd-even rows with the gfx950 permlane swaps,
// m = 8 / 4 pair mirror lanes (DPP row_mirror / row_half_mirror), m = 2 / 1
// use DPP quad permutes. For a reduction only the pairing between the two
// halves of each 2m-block matters, so mirror partners serve like xor ones.

__device__ __forceinline__ float partner(float v, uint32_t m, uint32_t lane) {
    const uint32_t u = __float_as_uint(v);
    switch (m) {
    case 32: {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __uint_as_float((lane & 32u) ? r[0] : r[1]);
    }
    case 16: {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float((lane & 16u) ? r[0] : r[1]);
    }
    case 8: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0x140, 0xf, 0xf, false));
    case 4: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0x141, 0xf, 0xf, false));
    case 2: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0x4e, 0xf, 0xf, false));
    default: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0xb1, 0xf, 0xf, false));
    }
}

// log2 of a power of two that is a compile-time constant after inlining.
__host__ __device__ constexpr int ilog2(uint32_t v) { return v <= 1 ? 0 : 1 + ilog2(v >> 1); }

// Sum over aligned groups of G lanes (G a power of two <= 64); every lane of
// a group receives the sum. The loops below run a constant number of times so
// they unroll into fixed DPP / permlane exchanges.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int i = 1; i <= ilog2(G); i++) v += partner(v, (uint32_t)G >> i, lane);
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave, without LDS traffic:
// Hillis-Steele steps 1, 2, 4, 8 inside each 16-lane row (DPP row_shr:n;
// lanes with no source n places back in their row add 0), then each row adds
// the totals of the rows before it (lanes 15, 31, 47 read as scalars).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v, uint32_t lane) {
    v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xf, 0xf, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xf, 0xf, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xf, 0xf, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xf, 0xf, false);   // row_shr:8
    const uint32_t t0 = __builtin_amdgcn_readlane(v, 15), t1 = __builtin_amdgcn_readlane(v, 31),
                   t2 = __builtin_amdgcn_readlane(v, 47);
    const uint32_t row = lane >> 4;
    return v + (row >= 1 ? t0 : 0u) + (row >= 2 ? t1 : 0u) + (row >= 3 ? t2 : 0u);
}

// Reduce-scatter: each lane holds S partial sums v[0..S) (one per row step)
// of a group of G lanes (S <= G). Returns the full group sum of step
// s = (lane & (G-1)) >> log2(G/S); all lanes of each G/S sub-group get it.
// G is a compile-time constant so every lane exchange is a fixed DPP /
// permlane instruction.
template <int S, int G>
__device__ __forceinline__ float reduce_scatter_k(float (&v)[S]) {
    const uint32_t lane = threadIdx.x & 63u;
    float w[S];
#pragma unroll
    for (int i = 0; i < S; i++) w[i] = v[i];
#pragma unroll
    for (int st = 1; st <= ilog2(S); st++) {   // S/2, S/4, .. values remain
        const uint32_t m = (uint32_t)G >> st;
        const int n = S >> st;
        const bool up = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < n; i++) {
            const float a = w[i], b = w[i + n];
            w[i] = (up ? b : a) + partner(up ? a : b, m, lane);
        }
    }
    float r = w[0];
#pragma unroll
    for (int st = ilog2(S) + 1; st <= ilog2(G); st++) r += partner(r, (uint32_t)G >> st, lane);
    return r;
}

// The same for a run-time group size g in {8, 16, 32, 64}.
template <int S>
__device__ __forceinline__ float reduce_scatter_c(float (&v)[S], uint32_t g) {
    switch (g) {
    case 64: return reduce_scatter_k<S, 64>(v);
    case 32: return reduce_scatter_k<S, 32>(v);
    case 16: return reduce_scatter_k<S, 16>(v);
    default: return reduce_scatter_k<S, 8>(v);
    }
}

template <int S>
__device__ __forceinline__ uint32_t scatter_step(uint32_t lane, uint32_t g) {
    return S == 1 ? 0u : (lane & (g - 1)) / (g / S);
}

// ---- routing ---------------------------------------------------------------------

// Order-preserving 32-bit key of a logit: unsigned key order equals float
// order (-0 folded into +0, which compare equal). Ties between equal logits
// are broken by index separately (lowest index wins). NaN logits take qw6's
// meaning (each round of qw6_cpu_moe_route scans with a strict '>' from
// best = index 0): a NaN at index 0 wins the first round whatever else is
// there (key 0xffffffff, above every other key), a NaN elsewhere never wins
// a comparison, so it is below every real key, -inf included (key 0).
__device__ __forceinline__ uint32_t route_key(float v, bool first) {
    if (v != v) return first ? 0xffffffffu : 0u;
    const uint32_t u = __float_as_uint(v + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
constexpr uint32_t kKeyNegInf = 0x007fffffu;   // route_key(-inf)

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const uint32_t o = __float_as_uint(partner(__uint_as_float(v), 32u >> i, lane));
        v = o > v ? o : v;
    }
    return v;
}

// qw6's routing (qw6_cpu_moe_route, qw6.c:2796-2827) runs top_k rounds of
// argmax (strict >, scan from index 0, winner set to -inf): it takes the
// top_k logits ordered by (value desc, index asc), then a softmax over them
// in that order. Once only -inf is left, its scan picks index 0 for every
// remaining round. Logits without NaN give qw6's indices exactly here too.
// Lane l holds experts 4l .. 4l+3 as order-preserving keys.

// Keys of one token's logits (0 for the lanes past n: below every real key).
__device__ __forceinline__ void route_keys(const float* __restrict__ logits, uint32_t n,
                                           uint32_t (&k)[4]) {
    const uint32_t lane = threadIdx.x & 63u;
    if ((((uintptr_t)logits & 15u) == 0) && 4 * lane + 3 < n) {
        const float4 v = *(const float4*)(logits + 4 * lane);
        k[0] = route_key(v.x, lane == 0); k[1] = route_key(v.y, false);
        k[2] = route_key(v.z, false); k[3] = route_key(v.w, false);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            k[i] = 4 * lane + i < n ? route_key(logits[4 * lane + i], lane == 0 && i == 0) : 0u;
    }
}

// Ranked selection, slow path: top_k rounds of a wave maximum over the lane
// heads (each lane's keys sorted, stable); the lowest lane whose head equals
// the maximum holds the lowest index with that logit and pops its head.
// Writes the (key, index) of rank r to scr[32 + r] for r < top_k.
constexpr uint32_t kRouteScr = 128;   // routing scratch per wave (uint2)

__device__ __forceinline__ void route_rounds(uint32_t (&k)[4], uint32_t top_k, uint2* scr) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t id[4] = {0, 1, 2, 3};
    auto cx = [&](int p) {
        const bool sw = k[p + 1] > k[p];
        const uint32_t k0 = k[p], k1 = k[p + 1], i0 = id[p], i1 = id[p + 1];
        k[p] = sw ? k1 : k0; k[p + 1] = sw ? k0 : k1;
        id[p] = sw ? i1 : i0; id[p + 1] = sw ? i0 : i1;
    };
    cx(0); cx(1); cx(2); cx(0); cx(1); cx(0);
    for (uint32_t r = 0; r < top_k; r++) {
        const uint32_t m = wave_max_u32(k[0]);
        const uint64_t b = __ballot(k[0] == m);
        const uint32_t w = (uint32_t)__ffsll((unsigned long long)b) - 1u;
        const uint32_t e = 4 * w + (uint32_t)__builtin_amdgcn_readlane((int)id[0], (int)w);
        if (lane == w) {
            scr[32 + r] = make_uint2(~e, m);
            k[0] = k[1]; k[1] = k[2]; k[2] = k[3]; k[3] = 0u;
            id[0] = id[1]; id[1] = id[2]; id[2] = id[3];
        }
    }
}

// One wave routes one token (scr: kRouteScr uint2 of LDS private to the
// wave). Fast path: T = the minimum over 8 groups of 8 lanes of each group's
// largest key is at most the 8th-largest key (8 distinct keys are >= T), so
// the top_k <= 8 winners are among the keys >= T -- about 20 of 256 for
// router logits. Those candidates are compacted into LDS and each is ranked
// against all of them at once with one 64-bit compare of (key, ~index) per
// pair; more than 32 candidates take route_rounds.
//
// route_rank ranks the top_k <= 8 keys. Fast path (returns true): lanes l and l + 32 both
// hold candidate l (l < ncand) as me = (~index, key) and, in rank, how many
// candidates order above it, each lane comparing against 16 of the 32 slots.
// Slow path (more than 32 candidates, returns false): scr[32 + r] holds the
// (~index, key) of rank r for r < top_k after a wave barrier.
__device__ __forceinline__ bool route_rank(uint32_t (&k)[4], uint32_t top_k, uint2* scr,
                                           uint2& me2, uint32_t& rank, uint32_t& ncand) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t g = max(max(k[0], k[1]), max(k[2], k[3]));
#pragma unroll
    for (int i = 0; i < 3; i++) {   // group maxima over lanes 8q .. 8q+7
        const uint32_t o = __float_as_uint(partner(__uint_as_float(g), 1u << i, lane));
        g = o > g ? o : g;
    }
#pragma unroll
    for (int i = 3; i < 6; i++) {   // minimum over the 8 groups
        const uint32_t o = __float_as_uint(partner(__uint_as_float(g), 1u << i, lane));
        g = o < g ? o : g;
    }
    const uint32_t t = (uint32_t)__builtin_amdgcn_readfirstlane((int)g);
    bool c[4];
    uint32_t pos = 0;
    ncand = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        c[i] = k[i] >= t && k[i] != 0u;
        const uint64_t b = __ballot(c[i]);
        ncand += __popcll(b);
        pos += __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
    }
    if (ncand > 32) {
        route_rounds(k, top_k, scr);
        __builtin_amdgcn_wave_barrier();
        return false;
    }
    // candidates of lower lanes first, then this lane's in index order, into
    // slots [0, ncand); the other slots below 64 hold (0, 0), below every
    // candidate. Branch-free: a non-candidate writes its own discard slot
    // 64 + lane (the wave's LDS writes land in program order).
    scr[lane] = make_uint2(0u, 0u);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        scr[c[i] ? pos : 64u + lane] = make_uint2(~(4 * lane + (uint32_t)i), k[i]);
        pos += c[i] ? 1u : 0u;
    }
    __builtin_amdgcn_wave_barrier();
    const uint32_t h = lane >> 5, l = lane & 31u;
    me2 = scr[l];
    const uint64_t me = ((uint64_t)me2.y << 32) | me2.x;
    uint32_t r = 0;
#pragma unroll
    for (uint32_t m = 0; m < 16; m++) {
        const uint2 o2 = scr[16 * h + m];
        const uint64_t o = ((uint64_t)o2.y << 32) | o2.x;
        r += o > me ? 1u : 0u;
    }
    rank = r + __float_as_uint(partner(__uint_as_float(r), 32, lane));
    return true;
}

// wave_route_keys: lanes j < top_k leave the j-th selected expert and its gate
// weight in out_e[j] / out_w[j] (any memory). It takes the keys already loaded
// by route_keys, so a caller can issue that load before its other memory
// traffic.
__device__ __forceinline__ void wave_route_keys(uint32_t (&k)[4], uint32_t top_k, uint2* scr,
                                                uint32_t* out_e, float* out_w) {
    const uint32_t lane = threadIdx.x & 63u;
    uint2 me2;
    uint32_t rank, ncand;
    if (route_rank(k, top_k, scr, me2, rank, ncand)) {
        if (lane < ncand && rank < top_k) scr[32 + rank] = me2;
        __builtin_amdgcn_wave_barrier();
    }
    uint32_t e = 0;
    float v = -INFINITY;
    if (lane < top_k) {
        const uint2 me = scr[32 + lane];
        // only -inf (or NaN away from index 0) left: qw6 picks index 0, whose
        // logit has been set to -inf by then
        const bool live = me.y > kKeyNegInf;
        v = live ? key_value(me.y) : -INFINITY;
        e = live ? ~me.x : 0u;
    }
    const float mx = key_value(scr[32].y);   // rank 0 holds the maximum
    const float ex = lane < top_k ? expf(v - mx) : 0.f;
    float sum = ex;
    sum += partner(sum, 1, lane);
    sum += partner(sum, 2, lane);
    sum += partner(sum, 4, lane);
    if (lane < top_k) {
        out_e[lane] = e;
        out_w[lane] = ex / sum;
    }
}

// The expert of rank u < top_k alone (same selection as wave_route_keys, no
// gate weights), uniform across the wave.
__device__ __forceinline__ uint32_t wave_route_select(uint32_t (&k)[4], uint32_t top_k,
                                                      uint32_t u, uint2* scr) {
    const uint32_t lane = threadIdx.x & 63u;
    uint2 me2 = make_uint2(0u, 0u);
    uint32_t rank = 0xffffffffu, ncand = 0;
    uint32_t ix, key;
    if (route_rank(k, top_k, scr, me2, rank, ncand)) {
        // fewer than u + 1 candidates (NaN logits are never candidates): rank
        // u is taken when only -inf and NaN are left, and qw6 picks index 0
        const uint64_t b = __ballot(lane < ncand && rank == u);
        if (!b) return 0u;
        const int w = __ffsll((unsigned long long)b) - 1;
        ix = (uint32_t)__builtin_amdgcn_readlane((int)me2.x, w);
        key = (uint32_t)__builtin_amdgcn_readlane((int)me2.y, w);
    } else {
        const uint2 me = scr[32 + u];
        ix = (uint32_t)__builtin_amdgcn_readfirstlane((int)me.x);
        key = (uint32_t)__builtin_amdgcn_readfirstlane((int)me.y);
    }
    return key > kKeyNegInf ? ~ix : 0u;   // only -inf left: qw6 picks index 0
}

__device__ __forceinline__ void wave_route(const float* __restrict__ logits, uint32_t n,
                                           uint32_t top_k, uint2* scr, uint32_t* out_e,
                                           float* out_w) {
    uint32_t k[4];
    route_keys(logits, n, k);
    wave_route_keys(k, top_k, scr, out_e, out_w);
}

// ---- synthetic data hash (twin of qw6_amd/synth.py) ------------------------------

__host__ __device__ inline uint64_t sm_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t sm_stream_key(uint64_t seed, uint64_t stream) {
    const uint64_t k = sm_mix(seed + 0x632BE59BD9B4E019ull);
    return sm_mix(k ^ (stream * 0xD1B54A32D192ED03ull));
}
__host__ __device__ inline uint64_t sm_hash(uint64_t key, uint64_t i) {
    return sm_mix(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}
// Irwin-Hall(12) standard normal from hashes hidx, hidx+1, hidx+2.
__host__ __device__ inline float sm_normal(uint64_t key, uint64_t hidx) {
    int64_t s = 0;
    for (int t = 0; t < 3; t++) {
        const uint64_t h = sm_hash(key, hidx + t);
        for (int q = 0; q < 4; q++) s += (int64_t)((h >> (16 * q)) & 0xffffu);
    }
    return (float)(s - 393210) * (1.0f / 65536.0f);
}

}  // namespace qw6
