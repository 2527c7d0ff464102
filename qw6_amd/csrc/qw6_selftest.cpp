// qw6_selftest.cpp -- device self-test: known-answer inputs through the
// library's host operations, checked against closed forms computed here in
// double precision (the role of qw6_vk_selftest, qw6_vk.c:1514-2133).
//
// Each case builds GGUF blocks whose dequantised values are known exactly
// (unit scales, patterned codes, zero grid indices; distinct Q6_K scales
// under qw6's even-only rule; pseudo-random IQ blocks decoded here from the
// lattice tables of iq_grid_data.h), runs the HIP operation and compares
// with sum_c w[r][c] * x[c]. Prints one line per case.

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "iq_grid_data.h"
#include "qw6_hip.h"

namespace {

void put16(uint8_t* b, uint32_t off, uint16_t v) {
    b[off] = (uint8_t)(v & 0xff);
    b[off + 1] = (uint8_t)(v >> 8);
}

double max_diff(const std::vector<float>& y, const std::vector<double>& want) {
    double m = 0.0;
    for (size_t i = 0; i < y.size(); i++) m = std::max(m, fabs((double)y[i] - want[i]));
    return m;
}

int report(const char* name, int rc, double diff, double tol) {
    const bool ok = rc == 0 && diff <= tol;
    fprintf(stderr, "qw6_hip selftest: %-10s %s (max diff %.3g, tolerance %.3g)\n", name,
            ok ? "ok" : "FAILED", rc == 0 ? diff : -1.0, tol);
    return ok ? 0 : 1;
}

// K-quant blocks with d = 1, dmin = 0 and every sub-block scale 1: weight =
// code (Q4_K, Q5_K) or code - 32 (Q6_K).
int kquant_case(int quant, const char* name) {
    const uint32_t rows = 3, cols = 256;
    const uint32_t bb = quant == 7 ? 210 : quant == 6 ? 176 : 144;
    std::vector<uint8_t> w(rows * bb, 0);
    std::vector<float> x(cols);
    for (uint32_t c = 0; c < cols; c++) x[c] = (float)sin(0.031 * c) + 0.25f * (float)cos(0.017 * c);
    std::vector<double> want(rows, 0.0);
    for (uint32_t r = 0; r < rows; r++) {
        uint8_t* b = &w[r * bb];
        if (quant == 7) {
            put16(b, 208, 0x3C00);
            for (int j = 0; j < 16; j++) b[192 + j] = 1;
        } else {
            put16(b, 0, 0x3C00);
            for (int j = 0; j < 4; j++) b[4 + j] = 1;        // scales of sub-blocks 0-3
            for (int j = 0; j < 4; j++) b[12 + j] = 1;       // low nibbles: sub-blocks 4-7
        }
        for (uint32_t c = 0; c < cols; c++) {
            int qv;
            if (quant == 4) {   // Q4_K: 32-byte groups, low nibbles then high
                qv = (int)((r * 3 + c * 5 + 7) & 15);
                const uint32_t off = 16 + (c >> 6) * 32 + (c & 31);
                b[off] |= (uint8_t)((c >> 5) & 1 ? qv << 4 : qv);
            } else if (quant == 6) {   // Q5_K: plus the 5th bit in qh
                qv = (int)((r * 7 + c * 3 + 5) & 31);
                const uint32_t off = 48 + (c >> 6) * 32 + (c & 31);
                b[off] |= (uint8_t)((c >> 5) & 1 ? (qv & 15) << 4 : (qv & 15));
                if (qv & 16) b[16 + (c & 31)] |= (uint8_t)(1u << ((c >> 6) * 2 + ((c >> 5) & 1)));
            } else {   // Q6_K: 4 low bits in ql, 2 high bits in qh
                const uint32_t half = c >> 7, in = c & 127, lane = in & 31, quad = in >> 5;
                const uint32_t u = (r * 11 + c * 7 + 9) & 63;
                qv = (int)u - 32;
                const uint32_t ql = half * 64 + lane + ((quad & 1) ? 32 : 0);
                b[ql] |= (uint8_t)(quad < 2 ? (u & 15) : (u & 15) << 4);
                b[128 + half * 32 + lane] |= (uint8_t)(((u >> 4) & 3) << (quad * 2));
            }
            want[r] += (double)qv * x[c];
        }
    }
    std::vector<float> y(rows);
    int rc;
    if (quant == 4) rc = qw6_hip_matmul_q4k_host(w.data(), x.data(), y.data(), rows, cols);
    else if (quant == 6) rc = qw6_hip_matmul_q5k_host(w.data(), x.data(), y.data(), rows, cols);
    else rc = qw6_hip_matmul_q6k_host(w.data(), x.data(), y.data(), rows, cols);
    return report(name, rc, max_diff(y, want), 1e-2);
}

// IQ formats with every index zero: IQ2_XXS grid entry 0 is all 8s and the
// block weight d * 0.25 * (0.5 + 0) * 8 = d; IQ2_S d * 0.125 * 8 = d; IQ3_S
// grid entry 0 is all 1s and the scale (1 + 0): every weight is d.
int iq_case(int quant, const char* name) {
    const uint32_t bb = quant == 13 ? 66 : quant == 11 ? 82 : 110;
    const uint32_t rows = 3, cols = 256;
    std::vector<uint8_t> w(rows * bb, 0);
    const uint16_t dh[3] = {0x3C00, 0x3E00, 0x4000};   // 1, 1.5, 2
    const double dv[3] = {1.0, 1.5, 2.0};
    for (uint32_t r = 0; r < rows; r++) put16(&w[r * bb], 0, dh[r]);
    std::vector<float> x(cols);
    double sx = 0.0;
    for (uint32_t c = 0; c < cols; c++) {
        x[c] = (float)sin(0.029 * c) + 0.15f * (float)cos(0.017 * c);
        sx += x[c];
    }
    std::vector<double> want(rows);
    for (uint32_t r = 0; r < rows; r++) want[r] = dv[r] * sx;
    std::vector<float> y(rows);
    int rc;
    if (quant == 13) rc = qw6_hip_matmul_iq2xxs_host(w.data(), x.data(), y.data(), rows, cols);
    else if (quant == 11) rc = qw6_hip_matmul_iq2s_host(w.data(), x.data(), y.data(), rows, cols);
    else rc = qw6_hip_matmul_iq3s_host(w.data(), x.data(), y.data(), rows, cols);
    return report(name, rc, max_diff(y, want), 2e-2);
}

// Q6_K with 16 distinct signed sub-block scales, d = 0.5: qw6 applies
// scales[8 h + 2 k] to the whole 32-run k of half h (qw6.c:1567-1570), so
// the odd-indexed scales never count.
int q6k_scales_case() {
    const uint32_t rows = 2, cols = 512, bb = 210, nb = cols / 256;
    std::vector<uint8_t> w(rows * nb * bb, 0);
    std::vector<float> x(cols);
    for (uint32_t c = 0; c < cols; c++) x[c] = (float)cos(0.023 * c) - 0.3f * (float)sin(0.041 * c);
    std::vector<double> want(rows, 0.0);
    double scale = 0.0;
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t kb = 0; kb < nb; kb++) {
            uint8_t* b = &w[(r * nb + kb) * bb];
            put16(b, 208, 0x3800);   // d = 0.5
            int8_t sc[16];
            for (int j = 0; j < 16; j++) {
                sc[j] = (int8_t)((int)((r * 5 + kb * 3 + j * 7) % 23) - 11);
                b[192 + j] = (uint8_t)sc[j];
            }
            for (uint32_t i = 0; i < 256; i++) {
                const uint32_t half = i >> 7, in = i & 127, lane = in & 31, quad = in >> 5;
                const uint32_t u = (r * 13 + kb * 29 + i * 11 + 3) & 63;
                const uint32_t ql = half * 64 + lane + ((quad & 1) ? 32 : 0);
                b[ql] |= (uint8_t)(quad < 2 ? (u & 15) : (u & 15) << 4);
                b[128 + half * 32 + lane] |= (uint8_t)(((u >> 4) & 3) << (quad * 2));
                const double wv = 0.5 * sc[8 * half + 2 * quad] * ((double)u - 32.0);
                want[r] += wv * x[kb * 256 + i];
                scale = std::max(scale, fabs(wv * x[kb * 256 + i]) * cols);
            }
        }
    std::vector<float> y(rows);
    const int rc = qw6_hip_matmul_q6k_host(w.data(), x.data(), y.data(), rows, cols);
    return report("q6_k_scl", rc, max_diff(y, want), 1e-6 * scale);
}

uint32_t rd32(const uint8_t* b, uint32_t off) {
    return (uint32_t)b[off] | ((uint32_t)b[off + 1] << 8) | ((uint32_t)b[off + 2] << 16) |
           ((uint32_t)b[off + 3] << 24);
}
uint32_t parity7(uint32_t s) {
    uint32_t p = 0;
    for (int n = 0; n < 7; n++) p ^= (s >> n) & 1u;
    return p;
}
double sgn(uint32_t bits, int n) { return ((bits >> n) & 1u) ? -1.0 : 1.0; }
double iq2_level(uint16_t code, int n) { return (double)QW6_IQ2_LEVEL((code >> (2 * n)) & 3u); }
double iq3_level(uint16_t code, int n) { return (double)(2 * ((code >> (3 * n)) & 7u) + 1); }

// The 256 weights of one IQ block with scale d, from the block layouts and
// the lattice tables (qw6.c:1580-1672): IQ2_XXS 8-weight groups with a 7-bit
// sign index (the eighth sign makes the count of negatives even) and a
// 4-bit scale per 32; IQ2_S 10-bit grid indices (two high bits in qh),
// explicit sign bytes, 4-bit scales per 16; IQ3_S 9-bit indices into the
// 4-byte grid, sign bytes, 4-bit scales (1 + 2s) per 32.
void iq_weights(int quant, const uint8_t* b, double d, double* w) {
    for (int j = 0; j < 8; j++) {
        if (quant == 13) {
            const uint32_t aux0 = rd32(b, 2 + 8 * j), aux1 = rd32(b, 6 + 8 * j);
            const double db = d * (0.5 + (double)(aux1 >> 28)) * 0.25;
            for (int l = 0; l < 4; l++) {
                const uint16_t g = qw6_iq2xxs_codes[(aux0 >> (8 * l)) & 0xffu];
                const uint32_t s7 = (aux1 >> (7 * l)) & 127u, s = s7 | (parity7(s7) << 7);
                for (int n = 0; n < 8; n++) w[32 * j + 8 * l + n] = db * iq2_level(g, n) * sgn(s, n);
            }
        } else if (quant == 11) {
            const uint32_t qh = b[66 + j], sc = b[74 + j];
            for (int l = 0; l < 4; l++) {
                const uint32_t gi = b[2 + 4 * j + l] | ((qh << (8 - 2 * l)) & 0x300u);
                const uint32_t sg = b[34 + 4 * j + l];
                const double db = d * (0.5 + (double)(l < 2 ? sc & 15u : sc >> 4)) * 0.25;
                for (int n = 0; n < 8; n++)
                    w[32 * j + 8 * l + n] = db * iq2_level(qw6_iq2s_codes[gi], n) * sgn(sg, n);
            }
        } else {
            const uint32_t qh = b[66 + j], scb = b[106 + j / 2];
            const double db = d * (double)(1 + 2 * ((j & 1) ? scb >> 4 : scb & 15u));
            for (int l = 0; l < 4; l++) {
                const uint32_t i1 = b[2 + 8 * j + 2 * l] | ((qh << (8 - 2 * l)) & 256u);
                const uint32_t i2 = b[2 + 8 * j + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256u);
                const uint32_t sg = b[74 + 4 * j + l];
                for (int n = 0; n < 4; n++) {
                    w[32 * j + 8 * l + n] = db * iq3_level(qw6_iq3s_codes[i1], n) * sgn(sg, n);
                    w[32 * j + 8 * l + 4 + n] = db * iq3_level(qw6_iq3s_codes[i2], n) * sgn(sg, 4 + n);
                }
            }
        }
    }
}

// IQ blocks of pseudo-random bytes (every sign pattern, high index bit and
// scale nibble occurs), d = 0.25, 0.5, 0.75 per row.
int iq_random_case(int quant, const char* name) {
    const uint32_t bb = quant == 13 ? 66 : quant == 11 ? 82 : 110;
    const uint32_t rows = 3, cols = 1024, nb = cols / 256;
    std::vector<uint8_t> w(rows * nb * bb);
    uint64_t st = 0x9E3779B97F4A7C15ull ^ (uint64_t)quant;
    for (auto& v : w) {
        st = st * 6364136223846793005ull + 1442695040888963407ull;
        v = (uint8_t)(st >> 56);
    }
    const uint16_t dh[3] = {0x3400, 0x3800, 0x3A00};   // 0.25, 0.5, 0.75
    const double dv[3] = {0.25, 0.5, 0.75};
    std::vector<float> x(cols);
    for (uint32_t c = 0; c < cols; c++) x[c] = (float)sin(0.013 * c + 0.3) + 0.2f * (float)cos(0.07 * c);
    std::vector<double> want(rows, 0.0);
    double scale = 0.0, wb[256];
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t kb = 0; kb < nb; kb++) {
            uint8_t* b = &w[(r * nb + kb) * bb];
            put16(b, 0, dh[r]);
            iq_weights(quant, b, dv[r], wb);
            for (int i = 0; i < 256; i++) {
                want[r] += wb[i] * x[kb * 256 + i];
                scale = std::max(scale, fabs(wb[i] * x[kb * 256 + i]) * cols);
            }
        }
    std::vector<float> y(rows);
    int rc;
    if (quant == 13) rc = qw6_hip_matmul_iq2xxs_host(w.data(), x.data(), y.data(), rows, cols);
    else if (quant == 11) rc = qw6_hip_matmul_iq2s_host(w.data(), x.data(), y.data(), rows, cols);
    else rc = qw6_hip_matmul_iq3s_host(w.data(), x.data(), y.data(), rows, cols);
    return report(name, rc, max_diff(y, want), 1e-6 * scale);
}

int f32_case() {   // 7 x 19 dense, w = 0.01 (r - c)
    const uint32_t rows = 7, cols = 19;
    std::vector<float> w(rows * cols), x(cols), y(rows);
    std::vector<double> want(rows, 0.0);
    for (uint32_t c = 0; c < cols; c++) x[c] = (float)cos(0.2 * c);
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t c = 0; c < cols; c++) {
            w[r * cols + c] = 0.01f * ((float)r - (float)c);
            want[r] += (double)w[r * cols + c] * x[c];
        }
    const int rc = qw6_hip_matvec_f32_host(w.data(), x.data(), y.data(), rows, cols);
    return report("matvec_f32", rc, max_diff(y, want), 2e-5);
}

int silu_case() {   // n = 513: one partial workgroup
    const uint32_t n = 513;
    std::vector<float> g(n), u(n), y(n);
    std::vector<double> want(n);
    for (uint32_t i = 0; i < n; i++) {
        g[i] = (float)((double)i * 0.013 - 3.0);
        u[i] = (float)cos(0.07 * i);
        want[i] = (double)g[i] / (1.0 + exp(-(double)g[i])) * u[i];
    }
    const int rc = qw6_hip_silu_mul_host(g.data(), u.data(), y.data(), n);
    return report("silu_mul", rc, max_diff(y, want), 1e-5);
}

int route_case() {   // 32 logits with a tie: top-4 by (value desc, index asc)
    const uint32_t n = 32, k = 4;
    std::vector<float> lg(n);
    for (uint32_t i = 0; i < n; i++) lg[i] = (float)((i * 13) % 17) * 0.25f;
    std::vector<uint32_t> order(n);
    for (uint32_t i = 0; i < n; i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return lg[a] > lg[b]; });
    std::vector<uint32_t> idx(k);
    std::vector<float> w(k);
    const int rc = qw6_hip_moe_route_host(lg.data(), idx.data(), w.data(), n, k);
    double se = 0.0;
    for (uint32_t j = 0; j < k; j++) se += exp((double)lg[order[j]] - lg[order[0]]);
    std::vector<double> want(k);
    bool same = true;
    for (uint32_t j = 0; j < k; j++) {
        want[j] = exp((double)lg[order[j]] - lg[order[0]]) / se;
        same = same && idx[j] == order[j];
    }
    return report("moe_route", rc == 0 && same ? 0 : -1, max_diff(w, want), 1e-6);
}

int gather_case() {   // dim 257, top-8, shared weight 0.25
    const uint32_t dim = 257, k = 8;
    std::vector<float> eo(k * dim), wt(k), sh(dim), y(dim);
    std::vector<double> want(dim, 0.0);
    for (uint32_t j = 0; j < k; j++) wt[j] = 0.05f * (float)(j + 1);
    for (uint32_t i = 0; i < dim; i++) {
        sh[i] = (float)sin(0.01 * i);
        want[i] = 0.25 * sh[i];
        for (uint32_t j = 0; j < k; j++) {
            eo[j * dim + i] = (float)cos(0.003 * i * (j + 1));
            want[i] += (double)wt[j] * eo[j * dim + i];
        }
    }
    const int rc = qw6_hip_moe_gather_host(eo.data(), wt.data(), sh.data(), 0.25f, y.data(), dim, k);
    return report("moe_gather", rc, max_diff(y, want), 2e-5);
}

}  // namespace

extern "C" int qw6_hip_selftest(void) {
    int bad = 0;
    bad += f32_case();
    bad += kquant_case(4, "q4_k");
    bad += kquant_case(6, "q5_k");
    bad += kquant_case(7, "q6_k");
    bad += iq_case(13, "iq2_xxs");
    bad += iq_case(11, "iq2_s");
    bad += iq_case(9, "iq3_s");
    bad += q6k_scales_case();
    bad += iq_random_case(13, "iq2_xxs_r");
    bad += iq_random_case(11, "iq2_s_r");
    bad += iq_random_case(9, "iq3_s_r");
    bad += silu_case();
    bad += route_case();
    bad += gather_case();
    fprintf(stderr, "qw6_hip selftest: %s\n", bad ? "FAILED" : "all passed");
    return bad ? -1 : 0;
}
