// qw6_selftest.cpp -- device self-test: known-answer inputs through the
// library's host operations, checked against closed forms computed here in
// double precision (the role of qw6_vk_selftest, qw6_vk.c:1514-2133).
//
// Each case builds GGUF blocks whose dequantised values are known exactly
// (unit scales, patterned codes, zero grid indices), runs the HIP operation
// and compares with sum_c w[r][c] * x[c]. Prints one line per case.

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

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
    bad += silu_case();
    bad += route_case();
    bad += gather_case();
    fprintf(stderr, "qw6_hip selftest: %s\n", bad ? "FAILED" : "all passed");
    return bad ? -1 : 0;
}
