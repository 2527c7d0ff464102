/* qw6_oracle.c -- CPU restatement of qw6's MoE FFN path (test infrastructure).
 *
 * The expected results for the HIP library: only tests, the smoke check and
 * the CPU-baseline leg of the benchmark use it. See qw6_oracle.h.
 *
 * Blocks are read through byte offsets of the GGUF layouts (little-endian,
 * 256 weights per super-block); the fp32 expressions keep the reference's
 * operand order so results are bit-identical under -ffp-contract=off.
 */
#include "qw6_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../qw6_amd/csrc/iq_grid_data.h"

#define QK 256

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}

/* ---- IQ tables: expanded from the packed codes ---------------------------- */

static uint64_t g_iq2xxs[256];
static uint64_t g_iq2s[1024];
static uint32_t g_iq3s[512];
static uint8_t g_ksigns[128];
static int g_tables_ready;

static uint64_t expand_iq2(uint16_t code) {
    uint64_t v = 0;
    for (int j = 0; j < 8; j++)
        v |= (uint64_t)QW6_IQ2_LEVEL((code >> (2 * j)) & 3) << (8 * j);
    return v;
}

static uint32_t expand_iq3(uint16_t code) {
    uint32_t v = 0;
    for (int j = 0; j < 4; j++) v |= (uint32_t)(2 * ((code >> (3 * j)) & 7) + 1) << (8 * j);
    return v;
}

static void tables_init(void) {
    if (g_tables_ready) return;
    for (int i = 0; i < 256; i++) g_iq2xxs[i] = expand_iq2(qw6_iq2xxs_codes[i]);
    for (int i = 0; i < 1024; i++) g_iq2s[i] = expand_iq2(qw6_iq2s_codes[i]);
    for (int i = 0; i < 512; i++) g_iq3s[i] = expand_iq3(qw6_iq3s_codes[i]);
    /* ksigns_iq2xs (qw6_iq_tables.h:11): 7 sign bits plus an 8th bit that
     * makes the total number of negative signs even. */
    for (int i = 0; i < 128; i++)
        g_ksigns[i] = (uint8_t)(i | ((__builtin_popcount((unsigned)i) & 1) << 7));
    g_tables_ready = 1;
}

void orc_iq_tables(uint64_t *iq2xxs, uint64_t *iq2s, uint32_t *iq3s,
                   uint8_t *ksigns, uint8_t *kmask) {
    tables_init();
    memcpy(iq2xxs, g_iq2xxs, sizeof(g_iq2xxs));
    memcpy(iq2s, g_iq2s, sizeof(g_iq2s));
    memcpy(iq3s, g_iq3s, sizeof(g_iq3s));
    memcpy(ksigns, g_ksigns, sizeof(g_ksigns));
    for (int j = 0; j < 8; j++) kmask[j] = (uint8_t)(1u << j);
}

/* ---- scalar helpers -------------------------------------------------------- */

/* Exact IEEE binary16 -> binary32 (qw6.c:1448-1471): subnormal halves are
 * renormalised, inf/NaN keep their payload. */
float orc_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        /* value = m * 2^-24; shift the leading one up to bit 10 */
        int shift = 0;
        while (!(m & 0x400u)) { m <<= 1; shift++; }
        bits = sign | ((uint32_t)(113 - shift) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static float bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* 6-bit (scale, min) of sub-block j from the 12 packed bytes of a Q4_K/Q5_K
 * block (qw6.c:1480-1490). */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

size_t orc_block_bytes(int quant) {
    switch (quant) {
    case ORC_Q_Q4_K_M: case ORC_Q_Q4_K_S: return 144;
    case ORC_Q_Q5_K: return 176;
    case ORC_Q_Q6_K: return 210;
    case ORC_Q_IQ2_XXS: return 66;
    case ORC_Q_IQ2_S: return 82;
    case ORC_Q_IQ3_S: return 110;
    default: return 0;
    }
}

size_t orc_row_bytes(int quant, uint32_t cols) {
    if (quant == ORC_Q_FP32) return (size_t)cols * 4;
    if (quant == ORC_Q_FP16 || quant == ORC_Q_BF16) return (size_t)cols * 2;
    size_t bb = orc_block_bytes(quant);
    if (!bb || cols % QK) return 0;
    return (size_t)(cols / QK) * bb;
}

/* ---- block decoders ------------------------------------------------------- */

/* Q4_K, 144 B: d@0 dmin@2 scales@4[12] qs@16[128] (qw6.c:1406-1411, 1492-1516).
 * Per 64 weights g: low nibbles of qs[32g..32g+31] use sub-block 2g, high
 * nibbles sub-block 2g+1; w = (d*sc)*q - dmin*m. */
static void deq_q4k(const uint8_t *b, float *y) {
    const float d = orc_fp16_to_f32(rd16(b));
    const float dmin = orc_fp16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4;
    const uint8_t *q = b + 16;
    for (int g = 0; g < 4; g++) {
        uint8_t s0, m0, s1, m1;
        orc_scale_min_k4(2 * g, sc, &s0, &m0);
        orc_scale_min_k4(2 * g + 1, sc, &s1, &m1);
        const float da = d * s0, ma = dmin * m0;
        const float db = d * s1, mb = dmin * m1;
        for (int l = 0; l < 32; l++) y[64 * g + l] = da * (q[32 * g + l] & 0x0f) - ma;
        for (int l = 0; l < 32; l++) y[64 * g + 32 + l] = db * (q[32 * g + l] >> 4) - mb;
    }
}

/* Q5_K, 176 B: d@0 dmin@2 scales@4[12] qh@16[32] qs@48[128]
 * (qw6.c:1413-1419, 1518-1548). As Q4_K plus a fifth bit from qh: bit 2g for
 * the low nibbles of group g, bit 2g+1 for the high nibbles. */
static void deq_q5k(const uint8_t *b, float *y) {
    const float d = orc_fp16_to_f32(rd16(b));
    const float dmin = orc_fp16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4;
    const uint8_t *qh = b + 16;
    const uint8_t *q = b + 48;
    for (int g = 0; g < 4; g++) {
        uint8_t s0, m0, s1, m1;
        orc_scale_min_k4(2 * g, sc, &s0, &m0);
        orc_scale_min_k4(2 * g + 1, sc, &s1, &m1);
        const float da = d * s0, ma = dmin * m0;
        const float db = d * s1, mb = dmin * m1;
        const uint8_t blo = (uint8_t)(1u << (2 * g)), bhi = (uint8_t)(2u << (2 * g));
        for (int l = 0; l < 32; l++)
            y[64 * g + l] = da * ((q[32 * g + l] & 0x0f) + (qh[l] & blo ? 16 : 0)) - ma;
        for (int l = 0; l < 32; l++)
            y[64 * g + 32 + l] = db * ((q[32 * g + l] >> 4) + (qh[l] & bhi ? 16 : 0)) - mb;
    }
}

/* Q6_K, 210 B: ql@0[128] qh@128[64] int8 scales@192[16] d@208
 * (qw6.c:1421-1426, 1550-1578). Each 128-weight half h has ql[64h..],
 * qh[32h..]; weight 128h + 32k + l (k = 0..3) is the 6-bit value
 * (nibble | 2 qh bits) - 32, scaled by d * scales[8h + 2k] -- qw6 reads the
 * even scale of each 32-run for all 32 of its weights. */
static void deq_q6k(const uint8_t *b, float *y) {
    const float d = orc_fp16_to_f32(rd16(b + 208));
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int h = 0; h < 2; h++) {
        const uint8_t *ql = b + 64 * h;
        const uint8_t *qh = b + 128 + 32 * h;
        float *o = y + 128 * h;
        for (int l = 0; l < 32; l++) {
            const int v0 = ((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int v1 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int v2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int v3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            o[l] = d * sc[8 * h + 0] * v0;
            o[l + 32] = d * sc[8 * h + 2] * v1;
            o[l + 64] = d * sc[8 * h + 4] * v2;
            o[l + 96] = d * sc[8 * h + 6] * v3;
        }
    }
}

/* IQ2_XXS, 66 B: d@0 then 8 x (u32 grid bytes, u32 signs/scale) per 32
 * weights (qw6.c:1428-1431, 1580-1602). */
static void deq_iq2xxs(const uint8_t *b, float *y) {
    const float d = orc_fp16_to_f32(rd16(b));
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t *p = b + 2 + 8 * ib;
        const uint32_t aux1 = rd32(p + 4);
        const float db = d * (0.5f + (aux1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const uint64_t grid = g_iq2xxs[p[l]];
            const uint8_t signs = g_ksigns[(aux1 >> (7 * l)) & 127];
            for (int j = 0; j < 8; j++) {
                const uint8_t gv = (uint8_t)(grid >> (8 * j));
                *y++ = db * gv * (signs & (1u << j) ? -1.0f : 1.0f);
            }
        }
    }
}

/* IQ2_S, 82 B: d@0 qs@2[32] signs@34[32] qh@66[8] scales@74[8]
 * (qw6.c:1433-1438, 1604-1630). 10-bit grid index = qs | 2 bits of qh. */
static void deq_iq2s(const uint8_t *b, float *y) {
    const float d = orc_fp16_to_f32(rd16(b));
    const uint8_t *qs = b + 2, *sg = b + 34, *qh = b + 66, *sc = b + 74;
    for (int ib = 0; ib < 8; ib++) {
        const float db0 = d * (0.5f + (sc[ib] & 0x0f)) * 0.25f;
        const float db1 = d * (0.5f + (sc[ib] >> 4)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const float dl = l < 2 ? db0 : db1;
            const uint32_t gi = qs[4 * ib + l] | ((qh[ib] << (8 - 2 * l)) & 0x300);
            const uint64_t grid = g_iq2s[gi];
            const uint8_t signs = sg[4 * ib + l];
            for (int j = 0; j < 8; j++) {
                const uint8_t gv = (uint8_t)(grid >> (8 * j));
                *y++ = dl * gv * (signs & (1u << j) ? -1.0f : 1.0f);
            }
        }
    }
}

/* IQ3_S, 110 B: d@0 qs@2[64] qh@66[8] signs@74[32] scales@106[4]
 * (qw6.c:1440-1446, 1632-1672). Per 32 weights ib: eight 4-byte grid entries
 * with a 9th index bit from qh[ib]; scale d * (1 + 2 * nibble) where ib even
 * takes the low nibble of scales[ib/2], ib odd the high nibble. */
static void deq_iq3s(const uint8_t *b, float *y) {
    const float d = orc_fp16_to_f32(rd16(b));
    const uint8_t *qs = b + 2, *qh = b + 66, *sg = b + 74, *sc = b + 106;
    for (int ib = 0; ib < 8; ib++) {
        const int nib = (ib & 1) ? (sc[ib / 2] >> 4) : (sc[ib / 2] & 0x0f);
        const float db = d * (1 + 2 * nib);
        const uint8_t *q = qs + 8 * ib;
        for (int l = 0; l < 4; l++) {
            const uint32_t g1 = g_iq3s[q[2 * l] | ((qh[ib] << (8 - 2 * l)) & 256)];
            const uint32_t g2 = g_iq3s[q[2 * l + 1] | ((qh[ib] << (7 - 2 * l)) & 256)];
            const uint8_t signs = sg[4 * ib + l];
            for (int j = 0; j < 4; j++) {
                y[j] = db * (uint8_t)(g1 >> (8 * j)) * (signs & (1u << j) ? -1.0f : 1.0f);
                y[j + 4] = db * (uint8_t)(g2 >> (8 * j)) * (signs & (1u << (j + 4)) ? -1.0f : 1.0f);
            }
            y += 8;
        }
    }
}

/* Row addressing and quant dispatch (qw6.c:1674-1724). Returns -1 for quants
 * the reference CPU path cannot decode (Q8_0, IQ2_M, ...). */
int orc_dequant_row(int quant, const void *data, uint32_t cols, uint32_t row,
                    float *dst) {
    tables_init();
    if (quant == ORC_Q_FP32) {
        memcpy(dst, (const float *)data + (size_t)row * cols, (size_t)cols * 4);
        return 0;
    }
    if (quant == ORC_Q_FP16 || quant == ORC_Q_BF16) {
        const uint8_t *s = (const uint8_t *)data + (size_t)row * cols * 2;
        for (uint32_t i = 0; i < cols; i++)
            dst[i] = quant == ORC_Q_FP16 ? orc_fp16_to_f32(rd16(s + 2 * i))
                                         : bf16_to_f32(rd16(s + 2 * i));
        return 0;
    }
    const size_t bb = orc_block_bytes(quant);
    if (!bb || cols % QK) return -1;
    const uint8_t *src = (const uint8_t *)data + (size_t)row * (cols / QK) * bb;
    void (*dec)(const uint8_t *, float *);
    switch (quant) {
    case ORC_Q_Q4_K_M: case ORC_Q_Q4_K_S: dec = deq_q4k; break;
    case ORC_Q_Q5_K: dec = deq_q5k; break;
    case ORC_Q_Q6_K: dec = deq_q6k; break;
    case ORC_Q_IQ2_XXS: dec = deq_iq2xxs; break;
    case ORC_Q_IQ2_S: dec = deq_iq2s; break;
    default: dec = deq_iq3s; break;
    }
    for (uint32_t i = 0; i < cols / QK; i++) dec(src + i * bb, dst + (size_t)i * QK);
    return 0;
}

/* y[r] = sum_c deq(W[r])[c] * x[c], c ascending, fp32 product then fp32 add
 * (qw6.c:1769-1791). nthreads > 1 splits rows over OpenMP threads; each row
 * keeps the same summation order, so the result is bit-identical. */
int orc_matvec(float *out, const orc_mat_t *w, const float *x,
               uint32_t max_rows, int nthreads) {
    if (!out || !w || !x || !w->data || !w->rows || !w->cols) return -1;
    if (!orc_row_bytes(w->quant, w->cols)) return -1;
    uint32_t rows = w->rows;
    if (max_rows > 0 && max_rows < rows) rows = max_rows;
    tables_init();
    int fail = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) reduction(| : fail)
    {
        float *row = malloc((size_t)w->cols * sizeof(float));
        if (!row) {
            fail = 1;
        } else {
#pragma omp for schedule(static)
            for (uint32_t r = 0; r < rows; r++) {
                if (orc_dequant_row(w->quant, w->data, w->cols, r, row) != 0) {
                    fail = 1;
                    continue;
                }
                float acc = 0.0f;
                for (uint32_t c = 0; c < w->cols; c++) acc += row[c] * x[c];
                out[r] = acc;
            }
            free(row);
        }
    }
    return fail ? -1 : 0;
}

/* Top-k by k rounds of argmax (strict >, scan from index 0 so the lowest
 * index wins ties; the winner is set to -inf), then a softmax over the k
 * selected logits in selection order (qw6.c:2796-2827). */
void orc_moe_route(int *idx, float *weights, const float *logits,
                   int n_experts, int top_k) {
    float v[256];
    memcpy(v, logits, (size_t)n_experts * sizeof(float));
    for (int k = 0; k < top_k; k++) {
        int best = 0;
        float bv = v[0];
        for (int i = 1; i < n_experts; i++)
            if (v[i] > bv) { bv = v[i]; best = i; }
        idx[k] = best;
        weights[k] = bv;
        v[best] = -INFINITY;
    }
    float mx = weights[0];
    for (int k = 1; k < top_k; k++)
        if (weights[k] > mx) mx = weights[k];
    float sum = 0.0f;
    for (int k = 0; k < top_k; k++) {
        weights[k] = expf(weights[k] - mx);
        sum += weights[k];
    }
    for (int k = 0; k < top_k; k++) weights[k] /= sum;
}

/* RMSNorm (qw6.c:2503-2513): ss = sum x^2 in order; s = 1/sqrtf(ss/n + eps);
 * out = x * s * w. */
void orc_rmsnorm(float *out, const float *x, const float *w, int dim, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < dim; i++) ss += x[i] * x[i];
    ss = 1.0f / sqrtf(ss / dim + eps);
    for (int i = 0; i < dim; i++) out[i] = x[i] * ss * w[i];
}

/* qw6.h:292-297 */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* mid = silu(gate) * up (qw6.c:2258; vulkan/silu_mul.comp). */
void orc_silu_mul(const float *gate, const float *up, float *out, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) out[i] = orc_silu(gate[i]) * up[i];
}

/* qw6_cpu_argmax (qw6.c:2858-2863): a running maximum that only a strictly
 * greater value replaces, so ties keep the lowest index, NaNs are never
 * taken, and a NaN at index 0 is never replaced. */
int orc_argmax(const float *x, int n) {
    int best = 0;
    float bv = x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    }
    return best;
}

/* out[i] = sum_e w_e * E[e][i] (+ s * shared[i]) in expert order
 * (vulkan/moe_gather.comp; host wrapper qw6_vk.c:929-970). */
void orc_moe_gather(const float *expert_out, const float *expert_weights,
                    const float *shared_out, float shared_weight, float *out,
                    uint32_t dim, uint32_t top_k) {
    for (uint32_t i = 0; i < dim; i++) {
        float acc = 0.0f;
        for (uint32_t e = 0; e < top_k; e++)
            acc += expert_weights[e] * expert_out[(size_t)e * dim + i];
        if (shared_out) acc += shared_weight * shared_out[i];
        out[i] = acc;
    }
}

/* The MoE FFN for one token (qw6.c:2226-2290): router matvec -> top-k route
 * -> per selected expert (in selection order) gate, up, silu*up, down,
 * out += w_k * down -> shared expert last with weight sigmoid(shared_router.x)
 * or 1.0 when there is no shared router. */
int orc_moe_layer(float *out, int *idx_out, float *w_out,
                  const float *router, const float *logits_in,
                  const orc_mat_t *experts, const orc_mat_t *shared,
                  const float *shared_router, const float *x,
                  uint32_t hidden, uint32_t n_experts, uint32_t top_k,
                  int nthreads) {
    if (!out || !experts || !x || n_experts == 0 || n_experts > 256 ||
        top_k == 0 || top_k > n_experts || (!router && !logits_in))
        return -1;
    const uint32_t inter = experts[0].rows;
    float logits[256];
    float *gate = calloc(inter, sizeof(float));
    float *up = calloc(inter, sizeof(float));
    float *mid = calloc(inter, sizeof(float));
    float *tmp = calloc(hidden, sizeof(float));
    int idx[256];
    float w[256];
    int rc = (gate && up && mid && tmp) ? 0 : -1;

    memset(out, 0, hidden * sizeof(float));
    if (rc == 0) {
        if (router) {
            orc_mat_t r = {router, ORC_Q_FP32, n_experts, hidden};
            rc = orc_matvec(logits, &r, x, n_experts, nthreads);
        } else {
            memcpy(logits, logits_in, n_experts * sizeof(float));
        }
    }
    if (rc == 0) {
        orc_moe_route(idx, w, logits, (int)n_experts, (int)top_k);
        for (uint32_t k = 0; k < top_k && rc == 0; k++) {
            const orc_mat_t *e = experts + 3 * (size_t)idx[k];
            rc = orc_matvec(gate, &e[0], x, e[0].rows, nthreads);
            if (rc == 0) rc = orc_matvec(up, &e[1], x, e[1].rows, nthreads);
            if (rc == 0) {
                for (uint32_t i = 0; i < e[0].rows; i++) mid[i] = orc_silu(gate[i]) * up[i];
                rc = orc_matvec(tmp, &e[2], mid, e[2].rows, nthreads);
            }
            if (rc == 0)
                for (uint32_t i = 0; i < hidden; i++) out[i] += w[k] * tmp[i];
        }
        if (idx_out) for (uint32_t k = 0; k < top_k; k++) idx_out[k] = idx[k];
        if (w_out) for (uint32_t k = 0; k < top_k; k++) w_out[k] = w[k];
    }
    if (rc == 0 && shared) {
        float sw = 1.0f;
        if (shared_router) {
            orc_mat_t r = {shared_router, ORC_Q_FP32, 1, hidden};
            rc = orc_matvec(&sw, &r, x, 1, 1);
            sw = orc_sigmoid(sw);
        }
        if (rc == 0) rc = orc_matvec(gate, &shared[0], x, shared[0].rows, nthreads);
        if (rc == 0) rc = orc_matvec(up, &shared[1], x, shared[1].rows, nthreads);
        if (rc == 0) {
            for (uint32_t i = 0; i < shared[0].rows; i++) mid[i] = orc_silu(gate[i]) * up[i];
            rc = orc_matvec(tmp, &shared[2], mid, shared[2].rows, nthreads);
        }
        if (rc == 0)
            for (uint32_t i = 0; i < hidden; i++) out[i] += sw * tmp[i];
    }
    free(gate); free(up); free(mid); free(tmp);
    return rc;
}
