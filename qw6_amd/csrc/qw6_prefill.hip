// qw6_prefill.hip -- the MoE FFN for a batch of tokens (prefill, batched
// verification) as grouped bf16-MFMA contractions on gfx950.
//
// qw6 runs its MoE block token by token (qw6_forward_token -> qw6_apply_layer_
// moe, qw6.c:2226-2290; qw6_prefill, qw6.c:2867-2882). With T tokens of top-8
// routing, expert e sees M_e of them; its gate/up/down are then T x K by K x N
// products over the M_e gathered rows. Kernels, in stream order:
//   k_pre_route   four waves per token: softmax top-k (wave_route), the
//                 shared-expert weight, the shared entries, the bf16 operands.
//   k_pre_sort    one workgroup: counting sort of the (token, k) pairs by
//                 expert into "entries", a tile list of <= 16 entries of
//                 one expert (the shared expert last, with every token), and
//                 the tiles grouped by the format of their gate/up and of
//                 their down matrix (experts may differ in format).
//   k_pre_gemm<0, F, FS> (one launch per format group, or per two groups
//                 of one occupancy class: the shared expert's own format
//                 beside the routed experts', or two routed formats)
//                 gate and up for 128 intermediate rows of one tile (64
//                 for Q6_K and IQ3_S): mid[entry] = silu(x.gate) * (x.up).
//   k_pre_gemm<1, F, FS> down for 256 hidden rows of one tile (128 for
//                 Q6_K and IQ3_S), times the entry's gate weight -> ybuf[entry].
//   k_pre_combine out[t] = sum_k ybuf[entry(t, k)] + ybuf[shared entry(t)]
//                 (+ residual), a fixed order: deterministic, no atomics.
//
// Numerics of the contraction (rel-L2 ~1e-5 against the fp32 CPU path):
//  - weights enter the MFMA as their integer codes (qw6_tile.h; the IQ
//    formats as their signed lattice values);
//  - activations enter as P bf16 parts, one MFMA each per 32-column
//    sub-block: hi + lo (hi = bf16(x), lo = bf16(x - hi)) for calls of
//    kPrefill3PartBelow tokens or more, hi + mid + lo (24 significant bits)
//    below that;
//  - the fp32 sub-block scale d*sc multiplies each sub-block's 16x16 MFMA
//    result; the code bias (128 or 160) and the K-quant minimum dmin*m, both
//    of the form (per-row integer) x (per-token sub-block sum of x), take one
//    more MFMA each per 256-column block: A holds the three bf16 parts of the
//    eight sub-block sums in k-slots 0-7, 8-15, 16-23, B the integers.
// Weight codes are decoded from the raw block bytes in LDS just before their
// MFMAs, two sub-blocks at a time, so a wave keeps 4 row tiles in flight.
// Sub-blocks are 32 columns in every format handled here (Q6_K under qw6's
// even-scale rule, qw6.c:1567-1570; IQ2_S's two 16-column scales take one
// MFMA pair each).

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qw6_dev.h"
#include "qw6_moe.h"
#include "qw6_tile.h"

namespace qw6 {
namespace {

__device__ const IqTables g_tabs_pre = make_tables();

constexpr uint32_t kPM = kPrefillTileEntries;   // entries per tile (one MFMA row group)
constexpr uint32_t kPWG = 256;    // threads per workgroup (4 waves)

// One float as P bf16 parts: P = 2: hi = bf16(x), lo = bf16(x - hi); P = 3:
// hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid). Returns the
// represented value (the parts' sum in fp32, in part order), which is what
// the MFMAs multiply and what the sub-block sums of the corrections add up.
template <int P>
__device__ __forceinline__ float split_parts(float x, __bf16& h, __bf16& m, __bf16& l) {
    h = (__bf16)x;
    const float r = x - (float)h;
    if (P == 2) {
        m = (__bf16)0.f;
        l = (__bf16)r;
        return (float)h + (float)l;
    }
    m = (__bf16)r;
    l = (__bf16)(r - (float)m);
    return ((float)h + (float)m) + (float)l;
}

// Eight floats -> their P bf16 parts, packed in MFMA operand order (m unused
// for P = 2); returns the sum of the represented values in fp32.
template <int P>
__device__ __forceinline__ float split8(const float (&v)[8], uint4& h, uint4& m, uint4& l) {
    uint32_t hw[4], mw[4], lw[4];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        __bf16 h0, m0, l0, h1, m1, l1;
        const float s0 = split_parts<P>(v[2 * i], h0, m0, l0);
        const float s1 = split_parts<P>(v[2 * i + 1], h1, m1, l1);
        sum += s0 + s1;
        hw[i] = bfb(h0) | (bfb(h1) << 16);
        mw[i] = bfb(m0) | (bfb(m1) << 16);
        lw[i] = bfb(l0) | (bfb(l1) << 16);
    }
    h = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    m = make_uint4(mw[0], mw[1], mw[2], mw[3]);
    l = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    return sum;
}

// ---- routing -----------------------------------------------------------------------

// One workgroup of four waves per token t: wave 0 routes it (wave_route);
// all four split its activations (into 3 bf16 parts for calls of fewer than
// kPrefill3PartBelow tokens, else 2) and take part in the shared-expert
// weight; thread 0 writes the shared entry.
constexpr uint32_t kRouteThreads = 256;
__global__ __launch_bounds__(kRouteThreads) void k_pre_route(PrefillLayer L, PrefillWs ws,
                                                             const float* __restrict__ xin,
                                                             const float* __restrict__ logits) {
    __shared__ uint2 scr[kRouteScr];
    __shared__ float red[kRouteThreads / 64];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const float* xr = xin + (size_t)t * L.hidden;
    if (wave == 0) {
        wave_route(logits + (size_t)t * L.n_experts, L.n_experts, L.top_k, scr,
                   ws.pidx + (size_t)t * L.top_k, ws.pw + (size_t)t * L.top_k);
        __builtin_amdgcn_wave_barrier();
        if (lane < L.top_k) {
            const size_t i = (size_t)t * L.top_k + lane;
            if (L.idx_out) L.idx_out[i] = ws.pidx[i];
            if (L.w_out) L.w_out[i] = ws.pw[i];
        }
    }
    if (L.shared_router) {   // sigmoid(shared_router . x) (qw6.c:2267-2285): per-thread, per-wave, then wave order
        float acc = 0.f;
        for (uint32_t c = tid; c < L.hidden; c += kRouteThreads) acc = fmaf(L.shared_router[c], xr[c], acc);
        acc = group_sum<64>(acc);
        if (lane == 0) red[wave] = acc;
    }
    // the token's bf16 hi / lo operands and its 32-column sums (lanes 4k .. 4k+3
    // hold one 32-column sub-block, 8 columns each)
    for (uint32_t c = tid; c < L.hidden / 8; c += kRouteThreads) {
        float v[8];
        const float4 a = ((const float4*)xr)[2 * c], b = ((const float4*)xr)[2 * c + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        uint4 h, m, l;
        float sum;
        const bool three = L.T < kPrefill3PartBelow;
        if (three) {
            sum = split8<3>(v, h, m, l);
            ((uint4*)(ws.xp[1] + (size_t)t * L.hidden))[c] = m;
        } else {
            sum = split8<2>(v, h, m, l);
        }
        ((uint4*)(ws.xp[0] + (size_t)t * L.hidden))[c] = h;
        ((uint4*)(ws.xp[three ? 2 : 1] + (size_t)t * L.hidden))[c] = l;
        sum += partner(sum, 1, lane);
        sum += partner(sum, 2, lane);
        if ((c & 3u) == 0) {
            const uint32_t sb = c >> 2;   // sub-block: block sb / 8, slot sb % 8
            uint16_t p3[3];
            split3(sum, p3);
            uint16_t* dst = ws.xs3 + ((size_t)t * (L.hidden / 256) + sb / 8) * 24 + sb % 8;
            dst[0] = p3[0]; dst[8] = p3[1]; dst[16] = p3[2];
        }
    }
    __syncthreads();   // red[] complete
    if (tid == 0) {
        float sw = 1.0f;
        if (L.shared_router) {
            float acc = 0.f;
#pragma unroll
            for (uint32_t w = 0; w < kRouteThreads / 64; w++) acc += red[w];
            sw = 1.0f / (1.0f + expf(-acc));
        }
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
    __shared__ uint8_t efmt[2][257];   // gate/up and down format per expert, the shared one last
    __shared__ uint32_t rel[2][257];   // per kind: an expert's first tile within its format group
    __shared__ uint32_t gst[2][F_NFMT];   // per kind: the groups' first places
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t ne = L.T * L.top_k, E = L.n_experts;
    // Every global load a thread needs goes out before its first wait: its
    // PT (token, k) pairs' experts and gate weights, and (expert tid) the
    // formats of expert tid's matrices. Layers beyond PT pairs per thread
    // reload per chunk.
    constexpr uint32_t PT = 4;
    const uint32_t chunk = PT * nthr;
    uint32_t ev[PT];
    float wv[PT];
#pragma unroll
    for (uint32_t u = 0; u < PT; u++) {
        const uint32_t i = u * nthr + tid;
        ev[u] = i < ne ? ws.pidx[i] : 0u;
        wv[u] = i < ne ? ws.pw[i] : 0.f;
    }
    if (tid <= E) {
        cnt[tid] = 0;
        efmt[0][tid] = tid == E ? L.sg.fmt : L.pk[0].regular ? L.pk[0].fmt : L.experts[tid].fmt[0];
        efmt[1][tid] = tid == E ? L.sd.fmt : L.pk[2].regular ? L.pk[2].fmt : L.experts[tid].fmt[2];
    }
    __syncthreads();
    for (uint32_t c0 = 0; c0 < ne; c0 += chunk) {
        if (c0) {
#pragma unroll
            for (uint32_t u = 0; u < PT; u++) {
                const uint32_t i = c0 + u * nthr + tid;
                ev[u] = i < ne ? ws.pidx[i] : 0u;
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < PT; u++)
            if (c0 + u * nthr + tid < ne) atomicAdd(&cnt[ev[u]], 1u);
    }
    __syncthreads();
    if (tid < 64) {   // exclusive scans of the counts and of the tiles per expert
        uint32_t run = 0, trun = 0;
        for (uint32_t e0 = 0; e0 < E; e0 += 64) {
            const uint32_t e = e0 + tid;
            const uint32_t c = e < E ? cnt[e] : 0u;
            const uint32_t nt = (c + kPM - 1) / kPM;
            const uint32_t sc = wave_scan_incl(c, tid), st = wave_scan_incl(nt, tid);
            if (e < E) { off[e] = run + sc - c; tof[e] = trun + st - nt; }
            run += __builtin_amdgcn_readlane(sc, 63);
            trun += __builtin_amdgcn_readlane(st, 63);
        }
        if (tid == 0) { off[E] = run; tof[E] = trun; }
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += nthr) cur[e] = off[e];
    __syncthreads();
    for (uint32_t c0 = 0; c0 < ne; c0 += chunk) {
        if (ne > chunk) {   // the registers hold the last chunk: reload
#pragma unroll
            for (uint32_t u = 0; u < PT; u++) {
                const uint32_t i = c0 + u * nthr + tid;
                ev[u] = i < ne ? ws.pidx[i] : 0u;
                wv[u] = i < ne ? ws.pw[i] : 0.f;
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < PT; u++) {
            const uint32_t i = c0 + u * nthr + tid;
            if (i >= ne) continue;
            const uint32_t pos = atomicAdd(&cur[ev[u]], 1u);
            if (pos >= ne) continue;   // cannot happen: the counts bound every expert's range
            ws.ent_tok[pos] = i / L.top_k;
            ws.ent_w[pos] = wv[u];
            ws.ent_pos[i] = pos;
        }
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
    if (tid == 0) {
        ws.n_tiles[0] = nrt;
        ws.n_tiles[1] = nsh;
    }
    // The tiles grouped by the format of their matrix, per matrix kind (wave
    // k: 0 gate/up, 1 down), each group in tile order (the tiles of one
    // expert stay together): one grouped launch per format (group pair).
    // With one routed format the list is grouped already (routed tiles, then
    // the shared expert's). Otherwise wave k finds each expert's place in its
    // group (experts, the shared one last, 64 to a round, a wave scan per
    // format present), then one thread per (kind, expert) writes its tiles.
    const uint32_t wave = tid >> 6, lane = tid & 63u;
    const uint32_t cap = prefill_tiles_max(L.T, L.top_k, L.n_experts);
    const bool mixed0 = __builtin_popcount(L.fmask_gu) > 1, mixed1 = __builtin_popcount(L.fmask_dn) > 1;
    if (wave < 2) {
        const int k = wave == 0 ? 0 : 2;
        uint32_t* order = ws.forder + (size_t)wave * cap;
        const uint32_t routed = k == 0 ? L.fmask_gu : L.fmask_dn;
        if (!(wave == 0 ? mixed0 : mixed1)) {
            const int fr = __builtin_ctz(routed);
            const int fs = nsh ? (int)efmt[wave][E] : -1;
            for (uint32_t i = lane; i < nrt + nsh; i += 64) order[i] = i;
            if (lane < F_NFMT) {
                uint32_t first = 0, count = 0;
                if ((int)lane == fr) count = nrt + (fs == fr ? nsh : 0u);
                else if ((int)lane == fs) { first = nrt; count = nsh; }
                ws.fseg[(wave * 8 + lane) * 2 + 0] = first;
                ws.fseg[(wave * 8 + lane) * 2 + 1] = count;
            }
        } else {
            const uint32_t present = routed | (nsh ? 1u << efmt[wave][E] : 0u);
            uint32_t base[F_NFMT];
#pragma unroll
            for (int f = 0; f < F_NFMT; f++) base[f] = 0;
            for (uint32_t e0 = 0; e0 <= E; e0 += 64) {
                const uint32_t e = e0 + lane;
                const uint32_t nt = e < E ? (cnt[e] + kPM - 1) / kPM : e == E ? nsh : 0u;
                const int f = e <= E ? (int)efmt[wave][e] : -1;
#pragma unroll
                for (int g = 0; g < F_NFMT; g++) {
                    if (!((present >> g) & 1u)) continue;
                    const uint32_t mine = f == g ? nt : 0u;
                    const uint32_t incl = wave_scan_incl(mine, lane);
                    if (f == g) rel[wave][e] = base[g] + incl - mine;   // place in the group
                    base[g] += __builtin_amdgcn_readlane(incl, 63);
                }
            }
            uint32_t run = 0;
#pragma unroll
            for (int f = 0; f < F_NFMT; f++) {
                if (lane == (uint32_t)f) {
                    gst[wave][f] = run;
                    ws.fseg[(wave * 8 + lane) * 2 + 0] = run;
                    ws.fseg[(wave * 8 + lane) * 2 + 1] = base[f];
                }
                run += base[f];
            }
        }
    }
    if (!mixed0 && !mixed1) return;   // the same for every thread
    __syncthreads();
    const uint32_t kk = tid >> 9, e = tid & 511u;
    if ((kk == 0 ? mixed0 : mixed1) && e <= E) {
        const uint32_t nt = e < E ? (cnt[e] + kPM - 1) / kPM : nsh;
        const uint32_t t0 = e < E ? tof[e] : nrt;
        const uint32_t o = gst[kk][efmt[kk][e]] + rel[kk][e];
        uint32_t* order = ws.forder + (size_t)kk * cap;
        for (uint32_t j = 0; j < nt; j++)
            if (o + j < cap) order[o + j] = t0 + j;
    }
}

// ---- the grouped contraction --------------------------------------------------------

// Shared memory of k_pre_gemm: the A operands of the tile for one 256-column
// block, operand-major so the operand reads (lane l reads 16 B at l) are
// conflict-free; then the raw weight block bytes of the workgroup's rows.
template <int P>
struct GemmLds {
    uint4 a[P][8][64];           // [part][sub-block][lane]: parts hi, (mid), lo
    float part[4][kPM];          // epilogue: per-wave sums of mid
    uint32_t raw[1];             // rows x raw_chunks(F) x 16 B
};

// LDS bytes of an IQ format's grid in the grouped kernels: bf16 entries,
// except IQ2_S's 1024 entries kept as their 8 byte values (8 KB).
__host__ __device__ constexpr uint32_t gemm_grid_bytes(int f) { return f == F_IQ2S ? 1024u * 8u : iq_grid_bytes(f); }
__device__ __forceinline__ uint2 u64_as_u2(uint64_t v) { return make_uint2((uint32_t)v, (uint32_t)(v >> 32)); }
// Eight byte values (v.x: values 0-3) as eight bf16: the float conversion of
// a byte is exact and so is its upper half for integers below 256.
__device__ __forceinline__ uint4 bytes_bf16(uint2 v) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t src = k < 2 ? v.x : v.y;
        const float f0 = ub(src, 2 * (k & 1)), f1 = ub(src, 2 * (k & 1) + 1);
        w[k] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    }
    return u4(w[0], w[1], w[2], w[3]);
}
template <int MODE, int F>
__host__ __device__ constexpr int gemm_rt() {   // row tiles per wave
    return (F == F_Q6K || F == F_IQ3S) ? 2 : 4;   // larger raw blocks: fewer rows
}

// The A operand parts of sub-block sb (this lane's), and one product of them
// with B: the parts' MFMAs chained into one fp32 accumulator, hi first.
template <int P>
struct AParts {
    uint4 v[P];
};
template <int P>
__device__ __forceinline__ AParts<P> a_parts(const GemmLds<P>& S, int sb, uint32_t lane) {
    AParts<P> a;
#pragma unroll
    for (int p = 0; p < P; p++) a.v[p] = S.a[p][sb][lane];
    return a;
}
template <int P>
__device__ __forceinline__ f32x4 mfma_parts(const AParts<P>& a, const uint4& b) {
    f32x4 c = mfma(a.v[0], b, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int p = 1; p < P; p++) c = mfma(a.v[p], b, c);
    return c;
}

// The products of one block for RT row tiles: acc[r] += sum over sub-blocks
// of d*sc * (codes . x), plus the bias / minimum corrections from one MFMA
// each against the 3-part sums (sxa: A operand, zero in lanes q = 3).
template <int F, int RT, int P>
__device__ __forceinline__ void gemm_block(const GemmLds<P>& S, const uint8_t* tab,
                                           const uint32_t (&R)[RT], uint32_t lane,
                                           const uint4& sxa, f32x4 (&acc)[RT]) {
    constexpr float bias = F == F_Q6K ? 160.f : 128.f;
    const uint32_t q = lane >> 4;
    if constexpr (F == F_IQ2XXS) {
        // Software pipeline over the sub-blocks: the grid reads of every row
        // tile are issued together (the signs are computed), and the 3 words
        // holding the next sub-block's 8 bytes (4 grid indices, 4 x 7 sign
        // bits, scale: bytes 2 + 8 sb of the 2-byte-aligned block) load while
        // this one's products run. db = d (0.5 + s) / 4 as one fma of exact terms.
        const uint4* grid = (const uint4*)tab;
        uint32_t wb[RT], sh[RT], w[RT][3];
        float d4[RT], d8[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const LdsRow row = lds_row(R[r]);
            const float d = h2f(rd16(S.raw, row, 0));
            d4[r] = 0.25f * d;
            d8[r] = 0.125f * d;
            wb[r] = row.w2;
            sh[r] = row.s2;
#pragma unroll
            for (int k = 0; k < 3; k++) w[r][k] = S.raw[wb[r] + k];
        }
#pragma unroll
        for (int sb = 0; sb < 8; sb++) {
            uint4 g[RT];
            uint32_t sg[RT];
            float db[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint32_t aux0 = __builtin_amdgcn_alignbyte(w[r][1], w[r][0], sh[r]);
                const uint32_t aux1 = __builtin_amdgcn_alignbyte(w[r][2], w[r][1], sh[r]);
                const uint32_t idx = (aux0 >> (8 * q)) & 255u;
                const uint32_t s7 = (aux1 >> (7 * q)) & 127u;
                g[r] = grid[idx];
                sg[r] = sign_pairs7(s7);
                db[r] = fmaf((float)(aux1 >> 28), d4[r], d8[r]);
            }
            __builtin_amdgcn_sched_barrier(0);
            const AParts<P> a = a_parts<P>(S, sb, lane);
            if (sb < 7) {
#pragma unroll
                for (int r = 0; r < RT; r++) {
#pragma unroll
                    for (int k = 0; k < 3; k++) w[r][k] = S.raw[wb[r] + 2 * (sb + 1) + k];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint4 b = apply_signs(g[r], sg[r]);
                const f32x4 c = mfma_parts<P>(a, b);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[r][j] = fmaf(db[r], c[j], acc[r][j]);
            }
        }
        return;
    }
    if constexpr (F == F_IQ3S) {
        // The same pipeline over IQ3_S's bytes, read as bytes (the LDS unit
        // extracts them): for group q of sub-block sb, grid index bytes
        // 2 + 8 sb + 2q, +1 (two 4-value entries), the high index bits at byte
        // 66 + sb (bits 2q, 2q + 1), the sign byte 74 + 4 sb + q and the scale
        // nibble of byte 106 + sb / 2; db = d (1 + 2 s) as one fma.
        const uint8_t* rb = (const uint8_t*)S.raw;
        const uint2* grid = (const uint2*)tab;
        uint32_t qa[RT], qb[RT], qh[RT], sg[RT], sc[RT];
        float d[RT], d2[RT];
        const uint32_t s1 = 8u - 2u * q, s2 = 7u - 2u * q;
        auto load = [&](int sb) {
#pragma unroll
            for (int r = 0; r < RT; r++) {
                qa[r] = rb[R[r] + 2 + 8 * sb + 2 * q];
                qb[r] = rb[R[r] + 3 + 8 * sb + 2 * q];
                qh[r] = rb[R[r] + 66 + sb];
                sg[r] = rb[R[r] + 74 + 4 * sb + q];
                if ((sb & 1) == 0) sc[r] = rb[R[r] + 106 + sb / 2];
            }
        };
#pragma unroll
        for (int r = 0; r < RT; r++) {
            d[r] = h2f(rd16(S.raw, lds_row(R[r]), 0));
            d2[r] = 2.f * d[r];
        }
        load(0);
#pragma unroll
        for (int sb = 0; sb < 8; sb++) {
            uint2 g1[RT], g2[RT];
            uint32_t y[RT];
            float db[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                g1[r] = grid[qa[r] | ((qh[r] << s1) & 256u)];
                g2[r] = grid[qb[r] | ((qh[r] << s2) & 256u)];
                y[r] = sign_pairs(sg[r]);
                const uint32_t nib = (sb & 1) ? sc[r] >> 4 : sc[r] & 15u;
                db[r] = fmaf((float)nib, d2[r], d[r]);
            }
            __builtin_amdgcn_sched_barrier(0);
            const AParts<P> a = a_parts<P>(S, sb, lane);
            if (sb < 7) load(sb + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint4 b = apply_signs(u4(g1[r].x, g1[r].y, g2[r].x, g2[r].y), y[r]);
                const f32x4 c = mfma_parts<P>(a, b);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[r][j] = fmaf(db[r], c[j], acc[r][j]);
            }
        }
        return;
    }
    if constexpr (F == F_IQ2S) {
        // The same pipeline over IQ2_S's bytes: for group q of sub-block sb,
        // the grid index byte 2 + 4 sb + q with bits 2q, 2q + 1 of byte
        // 66 + sb above it, the sign byte 34 + 4 sb + q, and byte 74 + sb
        // holding the scales of groups 0-1 (low nibble) and 2-3 (high). The
        // two scales take one MFMA pair each, over B with the other groups
        // zeroed; db = d (0.5 + s) / 4 as one fma.
        // The grid sits in LDS as its 8 byte values per entry (8 KB, so three
        // workgroups fit a CU) and widens to bf16 in registers.
        const uint8_t* rb = (const uint8_t*)S.raw;
        const uint2* grid = (const uint2*)tab;
        uint32_t qs[RT], qh[RT], sg[RT], sc[RT];
        float d4[RT], d8[RT];
        const uint32_t s1 = 8u - 2u * q;
        auto load = [&](int sb) {
#pragma unroll
            for (int r = 0; r < RT; r++) {
                qs[r] = rb[R[r] + 2 + 4 * sb + q];
                sg[r] = rb[R[r] + 34 + 4 * sb + q];
                qh[r] = rb[R[r] + 66 + sb];
                sc[r] = rb[R[r] + 74 + sb];
            }
        };
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const float d = h2f(rd16(S.raw, lds_row(R[r]), 0));
            d4[r] = 0.25f * d;
            d8[r] = 0.125f * d;
        }
        load(0);
#pragma unroll
        for (int sb = 0; sb < 8; sb++) {
            uint2 g[RT];
            uint32_t y[RT];
            float db[RT], db2[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                g[r] = grid[qs[r] | ((qh[r] << s1) & 0x300u)];
                y[r] = sign_pairs(sg[r]);
                db[r] = fmaf((float)(sc[r] & 15u), d4[r], d8[r]);
                db2[r] = fmaf((float)(sc[r] >> 4), d4[r], d8[r]);
            }
            __builtin_amdgcn_sched_barrier(0);
            const AParts<P> a = a_parts<P>(S, sb, lane);
            if (sb < 7) load(sb + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint4 b = apply_signs(bytes_bf16(g[r]), y[r]), z = u4(0, 0, 0, 0);
                const uint4 b0 = q < 2 ? b : z, b1 = q < 2 ? z : b;
                const f32x4 c = mfma_parts<P>(a, b0), c1 = mfma_parts<P>(a, b1);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[r][j] = fmaf(db2[r], c1[j], fmaf(db[r], c[j], acc[r][j]));
            }
        }
        return;
    }
    // K-quant formats (every IQ format returned above)
    TileScales ts[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        uint4 bsc, bmin;
        tile_scales<F>(S.raw, R[r], ts[r], bsc, bmin);
        const f32x4 u = mfma(sxa, bsc, f32x4{0.f, 0.f, 0.f, 0.f});
        const float cb = -bias * ts[r].d;
#pragma unroll
        for (int j = 0; j < 4; j++) acc[r][j] = fmaf(cb, u[j], acc[r][j]);
        if (F != F_Q6K) {
            const f32x4 v = mfma(sxa, bmin, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int j = 0; j < 4; j++) acc[r][j] = fmaf(-ts[r].dmin, v[j], acc[r][j]);
        }
    }
    // sub-blocks 2p, 2p + 1: one row tile's codes at a time (8 VGPRs live
    // instead of 8 RT), against the A operands of the two sub-blocks
#pragma unroll
    for (int p = 0; p < 4; p++) {
        AParts<P> a[2];
#pragma unroll
        for (int t = 0; t < 2; t++) a[t] = a_parts<P>(S, 2 * p + t, lane);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            uint4 b[2];
            tile_codes<F>(S.raw, R[r], q, p, b[0], b[1]);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const f32x4 c = mfma_parts<P>(a[t], b[t]);
                const float dsc = tile_dsc<F>(ts[r], 2 * p + t);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[r][j] = fmaf(dsc, c[j], acc[r][j]);
            }
        }
    }
}

// Registers of one 256-column block kb for k_pre_gemm's pipeline: this
// thread's NR raw 16-B pieces (pieces past a Q6_K block's end reload its first
// piece; the last piece of a block ends at most 15 bytes past it, inside the
// matrix, whose size -- a multiple of 256 rows of 16-byte-aligned blocks or of
// 420-byte Q6_K rows -- is a multiple of 16), its four A operand pieces and
// its part of the 3-part sums.
// Formats whose 256-column blocks are 16-byte aligned (Q4_K, Q5_K) address a
// piece as a 32-bit offset from its matrix, the matrix (gate or up) chosen by
// bit i of sel; the others keep a row pointer and piece index per load
// (their pieces depend on the block's alignment).
template <int F>
__host__ __device__ constexpr bool gemm_aligned() { return F == F_Q4K || F == F_Q5K; }

// A operand pieces (16 B) per thread and block: P parts x 8 sub-blocks x 64
// lanes over the workgroup's 256 threads. Thread (wave w, lane l) loads
// pieces u = NU w + i (i < NU): part u / 8, sub-block u % 8 of entry l % 16,
// columns 8 (l / 16) .. + 8; the pieces of a thread span at most two parts,
// whose rows are arow0 (part (NU w) / 8) and arow1 (the next part).
template <int P>
__host__ __device__ constexpr uint32_t a_pieces() { return 2 * P; }

template <int F, int P, uint32_t NR, uint32_t NP>
__device__ __forceinline__ void load_block(const uint8_t* const (&rowp)[NP],
                                           const uint32_t (&piece)[NR], const uint8_t* m0,
                                           const uint8_t* m1, uint32_t sel,
                                           const uint16_t* arow0, const uint16_t* arow1,
                                           const uint16_t* srow, uint32_t ua, uint32_t q,
                                           uint32_t kb, u32x4 (&rawv)[NR],
                                           u32x4 (&av)[a_pieces<P>()], u32x4& sxv) {
    constexpr uint32_t bb = fmt_block_bytes(F);
#pragma unroll
    for (uint32_t i = 0; i < NR; i++) {
        if constexpr (gemm_aligned<F>()) {   // piece[i]: byte offset of the piece at block 0
            const uint8_t* base = (sel >> i) & 1u ? m1 : m0;
            rawv[i] = ld_global<u32x4>(base + piece[i] + kb * bb);
        } else {
            const uint8_t* p = rowp[i] + (size_t)kb * bb;
            const uint32_t off = (uint32_t)((uintptr_t)p & 15u);
            const uint32_t ch = 16 * piece[i] < off + bb ? piece[i] : 0u;
            rawv[i] = ld_global<u32x4>(p - off + 16 * ch);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < a_pieces<P>(); i++) {
        const uint32_t u = ua + i;
        // (P = 2: the four pieces of a thread are in one part)
        const uint16_t* ar = P == 2 || (u >> 3) == (ua >> 3) ? arow0 : arow1;
        av[i] = *(const u32x4*)(ar + kb * 256 + 32 * (u & 7u) + 8 * q);
    }
    sxv = *(const u32x4*)(srow + kb * 24 + 8 * min(q, 2u));
}

// MODE 0: gate/up; wave w holds RT/2 gate tiles and the RT/2 up tiles of the
// same 8 RT intermediate rows (block rows: 32 RT). MODE 1: down; wave w holds
// RT tiles of 16 hidden rows (block rows: 64 RT). Work item (tile, row block).
// Software pipeline over the 256-column blocks: the raw weight bytes and the
// A operands of block kb + 1 are loaded into registers while block kb is
// multiplied, then written to LDS between two barriers.
// Occupancy class of a format's contraction: three workgroups per CU (at
// most 168 VGPRs; 53 KB of LDS or less each) except Q5_K, whose body needs
// up to 198 VGPRs (two). IQ2_S, with its grid kept as byte values, is in
// the three-workgroup class: at 168 VGPRs the gate/up launches whose first
// group is IQ2_S keep 3 dwords in scratch, and the down launches pairing
// Q4_K or IQ2_XXS with IQ2_S 5 (the others, IQ3_S + IQ2_S downs included,
// none). Format groups share a launch only within a
// class; a shared launch is built for its class, a single format's launch
// for three (Q4_K and IQ2_S) or with room for two (the others, whose
// allocations fit three workgroups per CU all the same).
__host__ __device__ constexpr int gemm_class(int f) { return f == F_Q5K ? 2 : 3; }
// Three activation parts (launches of fewer than kPrefill3PartBelow tokens)
// add 8 KB of A operands, so LDS fits two workgroups per CU: they take the
// register budget of two.
template <int F, int FS, int P>
__host__ __device__ constexpr int gemm_min_blocks() {
    return P == 3 ? 2
                  : F == FS ? ((F == F_Q4K || F == F_IQ2S) ? 3 : 2)
                            : (gemm_class(F) < gemm_class(FS) ? gemm_class(F) : gemm_class(FS));
}
template <int MODE, int F>
__host__ __device__ inline uint32_t gemm_ny(uint32_t hidden, uint32_t inter) {   // row blocks
    constexpr int RT = gemm_rt<MODE, F>();
    return MODE == 0 ? inter / (32 * RT) : hidden / (64 * RT);
}
template <int MODE, int F>
__host__ __device__ inline uint32_t gemm_rblocks(uint32_t hidden, uint32_t inter) {
    return gemm_ny<MODE, F>(hidden, inter);
}
// Workgroup slots of one XCD (32 CUs) for a format's occupancy class.
__host__ __device__ constexpr uint32_t gemm_slots_per_xcd(int f) { return 32u * (uint32_t)gemm_class(f); }
// A launch whose last group (FS) can run at half its row tiles per wave
// (gate/up: 4 -> 2, a gate and an up tile each; down: 2 -> 1, 4 -> 2) runs
// that group's last-round tiles so (k_pre_gemm).
template <int MODE, int F, int FS>
__host__ __device__ constexpr bool gemm_tail_split() {
    return MODE == 0 ? gemm_rt<MODE, FS>() == 4 : gemm_rt<MODE, FS>() >= 2;
}
// LDS row stride of the staged raw blocks in 16-byte chunks: one more than
// a row needs where that many would put the 16 rows of a row tile on two of
// the 64 banks (IQ3_S: 8 chunks, 128 bytes; 9 spread them over all 16).
__host__ __device__ constexpr uint32_t raw_stride(int f) { return raw_chunks(f) + (f == F_IQ3S ? 1u : 0u); }
template <int MODE, int F, int P>
__host__ __device__ constexpr size_t gemm_lds() {
    return offsetof(GemmLds<P>, raw) + (size_t)64 * gemm_rt<MODE, F>() * raw_stride(F) * 16 + gemm_grid_bytes(F);
}

// Row block yb of tile `tile` (format F), RT row tiles per wave, the
// activations in P bf16 parts.
template <int MODE, int F, int P, int RT = gemm_rt<MODE, F>()>
__device__ __forceinline__ void gemm_item(const PrefillLayer& L, const PrefillWs& ws, uint4 tile,
                                          uint32_t yb, uint8_t* smem) {
    GemmLds<P>& S = *(GemmLds<P>*)smem;
    const uint32_t mid_e = tile.x, ent0 = tile.y, cnt = tile.z;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t n = lane & 15u, q = lane >> 4;
    const bool shared = mid_e == L.n_experts;
    // Rows are addressed with format F's row bytes: the tile's expert must
    // hold format F (k_pre_sort groups the tiles so). The check keeps every
    // read inside the expert's own bytes whatever the grouping gave; the
    // item is uniform over the workgroup, so the return is too.
    {
        const int k = MODE == 0 ? 0 : 2;
        const int fe = shared ? (MODE == 0 ? L.sg.fmt : L.sd.fmt)
                              : L.pk[k].regular ? L.pk[k].fmt : L.experts[mid_e].fmt[k];
        if (fe != F) return;
    }
    const uint32_t K = MODE == 0 ? L.hidden : L.inter;
    const uint32_t nblk = K / 256;
    constexpr uint32_t NCH = raw_chunks(F);
    constexpr uint32_t bb = fmt_block_bytes(F);
    constexpr uint32_t ROWS = 64 * RT;            // weight rows staged per block
    constexpr uint32_t NC = ROWS * NCH;           // raw chunks per block
    constexpr uint32_t NR = (NC + kPWG - 1) / kPWG;   // raw chunks per thread (the last maybe none)
    constexpr uint32_t RS = raw_stride(F);        // LDS row stride in chunks
    // a thread without a last chunk loads its previous one again and does not store it
    const bool last = (NR - 1) * kPWG + tid < NC;
    const uint32_t rb = nblk * bb;
    const uint32_t r0 = yb * (MODE == 0 ? 32u * RT : 64u * RT);
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
    // staged row rr of the block: MODE 0 gate rows [0, ROWS/2), up rows after
    auto row_ptr = [&](uint32_t rr) -> const uint8_t* {
        if (MODE == 0)
            return rr < ROWS / 2 ? m0 + (size_t)(r0 + rr) * rb : m1 + (size_t)(r0 + rr - ROWS / 2) * rb;
        return m0 + (size_t)(r0 + rr) * rb;
    };
    uint32_t rrow[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        if (MODE == 0)
            rrow[r] = (r < RT / 2 ? 0u : ROWS / 2) + 8 * RT * wave + 16 * (r % (RT / 2)) + n;
        else
            rrow[r] = 16 * RT * wave + 16 * r + n;
    }

    // A operands: thread (wave w, lane l) loads pieces NU w .. NU w + NU - 1
    // (load_block) of entry l % 16 (clamped into the tile); the 3-part
    // sub-block sums of entry l % 16 (part l / 16)
    const uint32_t sm = min(n, cnt - 1);
    constexpr uint32_t NU = a_pieces<P>();
    const uint32_t ua = NU * (uint32_t)__builtin_amdgcn_readfirstlane(wave);
    const uint32_t pa = ua >> 3, pb = min(pa + 1, (uint32_t)P - 1);   // the thread's two parts
    const uint16_t* arow0;
    const uint16_t* arow1;
    const uint16_t* srow;
    if (MODE == 0) {
        const uint32_t tok = ws.ent_tok[ent0 + sm];
        arow0 = (pa == 0 ? ws.xp[0] : pa == 1 ? ws.xp[1] : ws.xp[2]) + (size_t)tok * L.hidden;
        arow1 = (pb == 0 ? ws.xp[0] : pb == 1 ? ws.xp[1] : ws.xp[2]) + (size_t)tok * L.hidden;
        srow = ws.xs3 + (size_t)tok * (L.hidden / 256) * 24;
    } else {
        arow0 = (pa == 0 ? ws.mp[0] : pa == 1 ? ws.mp[1] : ws.mp[2]) + (size_t)(ent0 + sm) * L.inter;
        arow1 = (pb == 0 ? ws.mp[0] : pb == 1 ? ws.mp[1] : ws.mp[2]) + (size_t)(ent0 + sm) * L.inter;
        srow = ws.ms3 + (size_t)(ent0 + sm) * (L.inter / 256) * 24;
    }
    constexpr bool kAl = gemm_aligned<F>();
    const uint8_t* rowp[kAl ? 1 : NR];   // this thread's raw pieces (see load_block)
    uint32_t piece[NR];
    uint32_t psel = 0;
#pragma unroll
    for (uint32_t i = 0; i < NR; i++) {
        uint32_t c = i * kPWG + tid;    // chunk: row c / NCH, 16-B piece c % NCH
        if (i + 1 == NR && !last) c -= kPWG;
        if constexpr (kAl) {
            const uint32_t rr = c / NCH;
            const bool up = MODE == 0 && rr >= ROWS / 2;
            piece[i] = (r0 + rr - (up ? ROWS / 2 : 0u)) * rb + 16 * (c % NCH);
            psel |= (up ? 1u : 0u) << i;
        } else {
            rowp[i] = row_ptr(c / NCH);
            piece[i] = c % NCH;
        }
    }
    if constexpr (kAl) rowp[0] = nullptr;
    u32x4 rawv[NR], av[NU], sxv;
    uint8_t* tab = (uint8_t*)S.raw + (size_t)ROWS * RS * 16;   // IQ lattice grid
    if constexpr (F == F_IQ2S) {   // the byte grid (visible after the loop's first barrier)
        for (uint32_t i = tid; i < 1024; i += kPWG) ((uint2*)tab)[i] = u64_as_u2(g_tabs_pre.iq2s[i]);
    } else if constexpr (is_iq(F)) {
        stage_iq_grid<F>(tab, g_tabs_pre, kPWG);
    }
    f32x4 acc[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    load_block<F, P, NR>(rowp, piece, m0, m1, psel, arow0, arow1, srow, ua, q, 0, rawv, av, sxv);
    for (uint32_t kb = 0; kb < nblk; kb++) {
        __syncthreads();   // every wave is done with block kb - 1's LDS data
#pragma unroll
        for (uint32_t i = 0; i < NR; i++) {
            const uint32_t c = i * kPWG + tid;
            if (i + 1 < NR || last) *(u32x4*)((uint8_t*)S.raw + 16u * (c / NCH * RS + c % NCH)) = rawv[i];
        }
#pragma unroll
        for (uint32_t i = 0; i < NU; i++) ((u32x4*)&S.a[0][0][0])[(ua + i) * 64 + lane] = av[i];
        const uint4 sxa = q < 3 ? u4(sxv.x, sxv.y, sxv.z, sxv.w) : u4(0, 0, 0, 0);
        if (kb + 1 < nblk)
            load_block<F, P, NR>(rowp, piece, m0, m1, psel, arow0, arow1, srow, ua, q, kb + 1, rawv, av, sxv);
        __syncthreads();   // block kb's bytes are in LDS
        uint32_t R[RT];
#pragma unroll
        for (int r = 0; r < RT; r++)
            R[r] = rrow[r] * RS * 16 +
                   (kAl ? 0u : (uint32_t)((uintptr_t)(row_ptr(rrow[r]) + (size_t)kb * bb) & 15u));
        gemm_block<F, RT, P>(S, tab, R, lane, sxa, acc);
    }

    // epilogue: lane holds entries 4 q + j of row n of its tiles
    if (MODE == 0) {
        // mid = silu(gate) * up as its P bf16 parts, plus the 32-row sums of mid:
        // wave w's 8 RT rows are part of sub-block (r0 + 8 RT w) / 32. Each
        // 16-row tile is summed over its lanes first and the tiles are added in
        // row order, so a sub-block's sum rounds the same for every tile shape.
        float part[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t m = 4 * q + j;
            float psum = 0.f;
#pragma unroll
            for (int r = 0; r < RT / 2; r++) {
                float hs = 0.f;
                if (m < cnt) {
                    const float gv = acc[r][j], uv = acc[r + RT / 2][j];
                    const float y = gv / (1.0f + expf(-gv)) * uv;
                    __bf16 h, md, l;
                    hs = split_parts<P>(y, h, md, l);
                    const size_t o = (size_t)(ent0 + m) * L.inter + r0 + 8 * RT * wave + 16 * r + n;
                    ws.mp[0][o] = __builtin_bit_cast(uint16_t, h);
                    if (P == 3) ws.mp[1][o] = __builtin_bit_cast(uint16_t, md);
                    ws.mp[P - 1][o] = __builtin_bit_cast(uint16_t, l);
                }
                psum += group_sum<16>(hs);   // over the 16 rows n of tile r
            }
            part[j] = psum;
        }
        if (n == 0) {
#pragma unroll
            for (int j = 0; j < 4; j++) S.part[wave][4 * q + j] = part[j];
        }
        __syncthreads();
        // sub-block sums: the 32 rows of a sub-block are 32 / (8 RT) waves' rows
        constexpr uint32_t WPS = 4 / RT;                  // waves per sub-block
        constexpr uint32_t NSB = 4 / WPS;                 // sub-blocks per block
        if (tid < NSB * kPM) {
            const uint32_t hh = tid / kPM, m = tid % kPM;
            if (m < cnt) {
                float v = 0.f;
#pragma unroll
                for (uint32_t w = 0; w < WPS; w++) v += S.part[WPS * hh + w][m];
                uint16_t p3[3];
                split3(v, p3);
                const uint32_t sbg = (r0 + 32 * hh) / 32;   // sub-block index in the row
                uint16_t* dst = ws.ms3 + ((size_t)(ent0 + m) * (L.inter / 256) + sbg / 8) * 24 + sbg % 8;
                dst[0] = p3[0]; dst[8] = p3[1]; dst[16] = p3[2];
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t m = 4 * q + j;
            if (m >= cnt) continue;
            const uint32_t e = ent0 + m;
            const float w = ws.ent_w[e];
#pragma unroll
            for (int r = 0; r < RT; r++)
                ws.ybuf[(size_t)e * L.hidden + r0 + 16 * RT * wave + 16 * r + n] = w * acc[r][j];
        }
    }
}

// One launch over the work items of one or two format groups (ws.forder,
// ws.fseg): group F's items and (FS != F) group FS's. Each workgroup takes
// one item and decodes it with its group's format; a layer whose shared
// expert has a format no routed expert has, or whose experts mix formats,
// needs no launch that fills only part of the GPU.
// XCD-aware work order: workgroup p runs on XCD p % 8 (round-robin
// dispatch), so XCD x takes the x-th contiguous range of each group's items
// (its slots first cover its range of F, then its range of FS) -- the row
// blocks of one tile (same A rows) and the tiles of one expert (same
// weights) then share that XCD's L2, and every XCD gets the same share of
// each format.
template <int MODE, int F, int FS, int P>
__global__ __launch_bounds__(kPWG, (gemm_min_blocks<F, FS, P>()))
void k_pre_gemm(PrefillLayer L, PrefillWs ws) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    if constexpr (gemm_tail_split<MODE, F, FS>()) {
        // The group dispatched last (FS) has its last-round tiles run as
        // items of half the rows (half the row tiles per wave), dispatched after
        // everything else: the last round of workgroup slots, which would
        // be part-empty, is filled by twice as many items of half the length.
        // Per XCD the slots run [F's items (F != FS)][FS at 4][FS at 2].
        const uint32_t cap = prefill_tiles_max(L.T, L.top_k, L.n_experts);
        const uint32_t first_f = ws.fseg[(MODE * 8 + F) * 2 + 0];
        const uint32_t n_f = F != FS ? ws.fseg[(MODE * 8 + F) * 2 + 1] : 0u;
        const uint32_t first = ws.fseg[(MODE * 8 + FS) * 2 + 0], n = ws.fseg[(MODE * 8 + FS) * 2 + 1];
        const uint32_t ny_f = gemm_ny<MODE, F>(L.hidden, L.inter);
        const uint32_t ny4 = gemm_rblocks<MODE, FS>(L.hidden, L.inter), ny2 = 2 * ny4;
        const uint32_t items_f = n_f * ny_f, pf = (items_f + 7) / 8;   // per XCD
        const uint32_t last = (pf + (n * ny4 + 7) / 8) % gemm_slots_per_xcd(gemm_class(F) < gemm_class(FS) ? F : FS);
        const uint32_t nb = min(n, last * 8 / ny4), na = n - nb;   // FS tiles at 4 / 2 row tiles per wave
        const uint32_t items_a = na * ny4, items_b = nb * ny2;
        const uint32_t pa = (items_a + 7) / 8, pb = (items_b + 7) / 8;
        const uint32_t slot = blockIdx.x / 8, xcd = blockIdx.x % 8;
        if (slot >= pf + pa + pb) return;
        const uint32_t seg = slot < pf ? 0u : slot < pf + pa ? 1u : 2u;
        const uint32_t it = seg == 0 ? xcd * pf + slot : seg == 1 ? xcd * pa + (slot - pf) : xcd * pb + (slot - pf - pa);
        if (it >= (seg == 0 ? items_f : seg == 1 ? items_a : items_b)) return;
        const uint32_t pos = seg == 0 ? first_f + it / ny_f : seg == 1 ? first + it / ny4 : first + na + it / ny2;
        const uint32_t oi = ws.forder[(size_t)MODE * cap + pos];
        if (oi >= ws.n_tiles[0] + ws.n_tiles[1]) return;   // not a tile of this call
        const uint4 tile = ws.tiles[oi];
        if constexpr (F != FS) {
            if (seg == 0) {
                gemm_item<MODE, F, P>(L, ws, tile, it % ny_f, smem);
                return;
            }
        }
        constexpr int RT = gemm_rt<MODE, FS>();
        if (seg == 2) gemm_item<MODE, FS, P, RT / 2>(L, ws, tile, it % ny2, smem);
        else gemm_item<MODE, FS, P, RT>(L, ws, tile, it % ny4, smem);
        return;
    }
    const uint32_t ny_a = gemm_ny<MODE, F>(L.hidden, L.inter);
    const uint32_t ny_b = gemm_ny<MODE, FS>(L.hidden, L.inter);
    const uint32_t first_a = ws.fseg[(MODE * 8 + F) * 2 + 0], n_a = ws.fseg[(MODE * 8 + F) * 2 + 1];
    const uint32_t first_b = FS != F ? ws.fseg[(MODE * 8 + FS) * 2 + 0] : 0u;
    const uint32_t n_b = FS != F ? ws.fseg[(MODE * 8 + FS) * 2 + 1] : 0u;
    const uint32_t items_a = n_a * ny_a, items_b = n_b * ny_b;
    const uint32_t pa = (items_a + 7) / 8, pb = (items_b + 7) / 8;   // per XCD
    const uint32_t slot = blockIdx.x / 8, xcd = blockIdx.x % 8;
    const bool in_b = slot >= pa;
    if (slot >= pa + pb) return;
    const uint32_t it = in_b ? xcd * pb + (slot - pa) : xcd * pa + slot;
    if (it >= (in_b ? items_b : items_a)) return;
    const uint32_t ny = in_b ? ny_b : ny_a;
    const uint32_t cap = prefill_tiles_max(L.T, L.top_k, L.n_experts);
    const uint32_t oi = ws.forder[(size_t)MODE * cap + (in_b ? first_b : first_a) + it / ny];
    if (oi >= ws.n_tiles[0] + ws.n_tiles[1]) return;   // not a tile of this call
    const uint4 tile = ws.tiles[oi];
    if constexpr (FS == F) {
        gemm_item<MODE, F, P>(L, ws, tile, it % ny, smem);
    } else {
        if (in_b) gemm_item<MODE, FS, P>(L, ws, tile, it % ny, smem);
        else gemm_item<MODE, F, P>(L, ws, tile, it % ny, smem);
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
    const uint32_t n4 = L.hidden / 4;
    for (uint32_t i = blockIdx.y * 256 + threadIdx.x; i < n4; i += 256 * gridDim.y) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (uint32_t k = 0; k < 8; k++)
            if (k < L.top_k) {
                const float4 y = ((const float4*)(ws.ybuf + (size_t)pos[k] * L.hidden))[i];
                v.x += y.x; v.y += y.y; v.z += y.z; v.w += y.w;
            }
        if (sh) {
            const float4 y = ((const float4*)(ws.ybuf + (size_t)se * L.hidden))[i];
            v.x += y.x; v.y += y.y; v.z += y.z; v.w += y.w;
        }
        if (L.residual) {
            const float4 r = ((const float4*)(L.residual + (size_t)t * L.hidden))[i];
            v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
        }
        ((float4*)(L.out + (size_t)t * L.hidden))[i] = v;
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
// NV = hidden / 256 float4 per lane, a template constant, so the router row
// and the four tokens' inputs are requested at once (one memory round trip).
template <int NV>
__global__ __launch_bounds__(64) void k_pre_router(const float* __restrict__ router,
                                                   const float* __restrict__ x, float* logits,
                                                   uint32_t n_experts, uint32_t T) {
    constexpr uint32_t hidden = 256 * NV;
    const uint32_t e = blockIdx.x, t0 = 4 * blockIdx.y, lane = threadIdx.x;
    const float4* wr = (const float4*)(router + (size_t)e * hidden);
    float4 w[NV], xv[4][NV];
#pragma unroll
    for (int i = 0; i < NV; i++) w[i] = wr[64 * i + lane];
#pragma unroll
    for (uint32_t t = 0; t < 4; t++) {
        const float4* xr = (const float4*)(x + (size_t)min(t0 + t, T - 1) * hidden);
#pragma unroll
        for (int i = 0; i < NV; i++) xv[t][i] = xr[64 * i + lane];
    }
#pragma unroll
    for (uint32_t t = 0; t < 4; t++) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            acc = fmaf(w[i].x, xv[t][i].x, acc); acc = fmaf(w[i].y, xv[t][i].y, acc);
            acc = fmaf(w[i].z, xv[t][i].z, acc); acc = fmaf(w[i].w, xv[t][i].w, acc);
        }
        const float v = group_sum<64>(acc);
        if (lane == 0 && t0 + t < T) logits[(size_t)(t0 + t) * n_experts + e] = v;
    }
}

template <int MODE, int F, int FS, int P>
void launch_gemm_ff(const PrefillLayer& L, const PrefillWs& ws, uint32_t cap, hipStream_t st) {
    const size_t lds = gemm_lds<MODE, F, P>() > gemm_lds<MODE, FS, P>() ? gemm_lds<MODE, F, P>()
                                                                        : gemm_lds<MODE, FS, P>();
    uint32_t ny_a = gemm_ny<MODE, F>(L.hidden, L.inter), ny_b = gemm_ny<MODE, FS>(L.hidden, L.inter);
    if (gemm_tail_split<MODE, F, FS>()) ny_b = 2 * ny_b;   // at most every FS tile at half the rows
    // at most cap tiles in all; the kernel maps workgroups to its groups'
    // items, per XCD a rounded-up share of each group
    const uint32_t nwg = (cap * (ny_a > ny_b ? ny_a : ny_b) + 7) / 8 * 8 +
                         (gemm_tail_split<MODE, F, FS>() ? 24u : FS != F ? 8u : 0u);
    k_pre_gemm<MODE, F, FS, P><<<nwg, kPWG, lds, st>>>(L, ws);
}
// Groups of one occupancy class only (no other pair is instantiated).
template <int MODE, int F, int FS, int P>
int launch_pair(const PrefillLayer& L, const PrefillWs& ws, uint32_t cap, hipStream_t st) {
    if constexpr (gemm_class(F) == gemm_class(FS)) {
        launch_gemm_ff<MODE, F, FS, P>(L, ws, cap, st);
        return 0;
    } else {
        return qw6_fail("batched path: formats %d and %d paired across occupancy classes", F, FS);
    }
}
template <int MODE, int F, int P>
int launch_gemm_f(int fs, const PrefillLayer& L, const PrefillWs& ws, uint32_t cap, hipStream_t st) {
    switch (fs) {
    case F_Q4K: return launch_pair<MODE, F, F_Q4K, P>(L, ws, cap, st);
    case F_Q5K: return launch_pair<MODE, F, F_Q5K, P>(L, ws, cap, st);
    case F_Q6K: return launch_pair<MODE, F, F_Q6K, P>(L, ws, cap, st);
    case F_IQ2XXS: return launch_pair<MODE, F, F_IQ2XXS, P>(L, ws, cap, st);
    case F_IQ2S: return launch_pair<MODE, F, F_IQ2S, P>(L, ws, cap, st);
    default: return launch_pair<MODE, F, F_IQ3S, P>(L, ws, cap, st);
    }
}

// The format groups of one matrix kind (routed formats `routed`, the shared
// expert's `fsh`, or -1), up to two to a launch: in the order the shared
// expert's group (when no routed expert has its format), then the routed
// groups by format, each group not yet launched takes the next one of its
// occupancy class as its partner. P: the activations' bf16 parts.
template <int MODE, int P>
int launch_gemm(uint32_t routed, int fsh, const PrefillLayer& L, const PrefillWs& ws, hipStream_t st) {
    const uint32_t cap = prefill_tiles_max(L.T, L.top_k, L.n_experts);
    int order[F_NFMT + 1], n = 0;
    bool done[F_NFMT + 1] = {};
    if (fsh >= 0 && !((routed >> fsh) & 1u)) order[n++] = fsh;
    for (int f = 0; f < F_NFMT; f++)
        if ((routed >> f) & 1u) order[n++] = f;
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        const int fa = order[i];
        int fb = fa;
        for (int j = i + 1; j < n; j++)
            if (!done[j] && gemm_class(order[j]) == gemm_class(fa)) {
                fb = order[j];
                done[j] = true;
                break;
            }
        int rc;
        switch (fa) {
        case F_Q4K: rc = launch_gemm_f<MODE, F_Q4K, P>(fb, L, ws, cap, st); break;
        case F_Q5K: rc = launch_gemm_f<MODE, F_Q5K, P>(fb, L, ws, cap, st); break;
        case F_Q6K: rc = launch_gemm_f<MODE, F_Q6K, P>(fb, L, ws, cap, st); break;
        case F_IQ2XXS: rc = launch_gemm_f<MODE, F_IQ2XXS, P>(fb, L, ws, cap, st); break;
        case F_IQ2S: rc = launch_gemm_f<MODE, F_IQ2S, P>(fb, L, ws, cap, st); break;
        default: rc = launch_gemm_f<MODE, F_IQ3S, P>(fb, L, ws, cap, st); break;
        }
        if (rc) return -1;
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return qw6_fail("batched kernel launch: %s", hipGetErrorString(e));
    }
    return 0;
}

}  // namespace

bool prefill_supports(int f) { return f >= F_Q4K && f <= F_IQ3S; }

int prefill_forward(const PrefillLayer& L, const PrefillWs& ws, hipStream_t st) {
    if (L.hidden % 256 || L.inter % 256)
        return qw6_fail("batched path needs hidden, inter multiples of 256");
    const uint32_t all = (1u << F_NFMT) - 1u;
    if (!L.fmask_gu || !L.fmask_dn || (L.fmask_gu & ~all) || (L.fmask_dn & ~all) ||
        (L.sg.p && (!prefill_supports(L.sg.fmt) || !prefill_supports(L.sd.fmt) ||
                    L.su.fmt != L.sg.fmt)))
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
        const dim3 g(L.n_experts, (L.T + 3) / 4);
        switch (L.hidden / 256) {
        case 1: k_pre_router<1><<<g, 64, 0, st>>>(L.router, xin, ws.logits, L.n_experts, L.T); break;
        case 2: k_pre_router<2><<<g, 64, 0, st>>>(L.router, xin, ws.logits, L.n_experts, L.T); break;
        case 4: k_pre_router<4><<<g, 64, 0, st>>>(L.router, xin, ws.logits, L.n_experts, L.T); break;
        case 8: k_pre_router<8><<<g, 64, 0, st>>>(L.router, xin, ws.logits, L.n_experts, L.T); break;
        default: return qw6_fail("batched router needs hidden in {256, 512, 1024, 2048}");
        }
        logits = ws.logits;
    }
    PrefillLayer Lx = L;
    Lx.x = xin;
    k_pre_route<<<L.T, kRouteThreads, 0, st>>>(Lx, ws, xin, logits);
    k_pre_sort<<<1, 1024, 0, st>>>(Lx, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qw6_fail("batched routing launch: %s", hipGetErrorString(e));
    // the activations' bf16 parts (k_pre_route split them the same way)
    if (L.T < kPrefill3PartBelow) {
        if (launch_gemm<0, 3>(L.fmask_gu, L.sg.p ? L.sg.fmt : -1, Lx, ws, st)) return -1;
        if (launch_gemm<1, 3>(L.fmask_dn, L.sg.p ? L.sd.fmt : -1, Lx, ws, st)) return -1;
    } else {
        if (launch_gemm<0, 2>(L.fmask_gu, L.sg.p ? L.sg.fmt : -1, Lx, ws, st)) return -1;
        if (launch_gemm<1, 2>(L.fmask_dn, L.sg.p ? L.sd.fmt : -1, Lx, ws, st)) return -1;
    }
    k_pre_combine<<<dim3(L.T, (L.hidden / 4 + 255) / 256), 256, 0, st>>>(Lx, ws);
    e = hipGetLastError();
    if (e != hipSuccess) return qw6_fail("batched combine launch: %s", hipGetErrorString(e));
    return 0;
}

}  // namespace qw6
