/* A C11 caller of the device API, built with qw6's own warning flags
 * (-std=c11 -Wall -Wextra -Werror -Wpedantic, the reference Makefile:5), as
 * qw6's C code would call the library in place of its Vulkan path:
 *
 *  1. qw6_vk_selftest through the compat header (qw6.c:3540,
 *     `qw6 --vulkan-self-test`), then the F32 host matvec probe
 *     (qw6.c:1877) on the self-test's 7 x 19 case against its closed form;
 *  2. the seeded MoE layer of the decode benchmark (hidden 2048, 256
 *     experts top-8, inter 512, Q4_K gate/up, Q6_K down, F32 router, a
 *     shared expert; seed 11, layer 0) generated on the device with
 *     qw6_hip_synth_*, its experts registered with qw6_hip_experts_create
 *     (the role of bind_expert_pack, qw6.c:542-597);
 *  3. one token through qw6_hip_moe_forward eagerly, then the same call
 *     captured with hipStreamBeginCapture into a HIP graph and replayed
 *     three times;
 *  4. every result against qw6's own qw6_apply_layer_moe output for that
 *     layer and token (raw little-endian files: idx int32[8], w f32[8],
 *     out f32[2048]): indices equal, weights within 2e-5, output rel-L2 <=
 *     1e-5.
 *
 *     qw6_layer_caller GOLDEN_DIR      (prints "ok" and exits 0 on success)
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qw6_hip_compat.h"

#define HIDDEN 2048u
#define INTER 512u
#define N_EXPERTS 256u
#define TOP_K 8u
#define SEED 11u

/* qw6_quant_t ids (qw6.h:76-91) and the generator's tensor kinds */
enum { Q4_K_M = 4, Q6_K = 7 };
enum { K_ROUTER = 1, K_GATE = 2, K_UP = 3, K_DOWN = 4, K_SGATE = 5, K_SUP = 6, K_SDOWN = 7, K_X = 8 };

static uint64_t stream_id(uint32_t layer, uint32_t kind, uint32_t expert) {
    return ((uint64_t)layer << 24) | ((uint64_t)kind << 16) | expert;
}

static int fails = 0;

#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            fprintf(stderr, "FAIL: " __VA_ARGS__);        \
            fprintf(stderr, " (%s)\n", qw6_hip_last_error()); \
            return 1;                                     \
        }                                                 \
    } while (0)
#define HIPCHECK(call)                                                          \
    do {                                                                        \
        hipError_t e_ = (call);                                                 \
        if (e_ != hipSuccess) {                                                 \
            fprintf(stderr, "FAIL: %s: %s\n", #call, hipGetErrorString(e_));    \
            return 1;                                                           \
        }                                                                       \
    } while (0)

static int read_file(const char *dir, const char *name, void *dst, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) return -1;
    const size_t n = fread(dst, 1, bytes, f);
    fclose(f);
    return n == bytes ? 0 : -1;
}

/* the generated layer's row bytes: cols / 256 blocks of 144 (Q4_K) or 210 (Q6_K) */
static size_t matrix_bytes(int quant, uint32_t rows, uint32_t cols) {
    return (size_t)rows * (cols / 256u) * (quant == Q6_K ? 210u : 144u);
}

/* One expert pack: n_experts matrices of one kind, expert e at base + e * bytes. */
static int make_pack(qw6_hip_ctx_t *ctx, int quant, uint32_t kind, uint32_t rows, uint32_t cols,
                     qw6_hip_matrix_t *mats) {
    const size_t bytes = matrix_bytes(quant, rows, cols);
    void *base = NULL;
    if (qw6_hip_alloc(ctx, bytes * N_EXPERTS, &base)) return -1;
    for (uint32_t e = 0; e < N_EXPERTS; e++) {
        uint8_t *p = (uint8_t *)base + (size_t)e * bytes;
        if (qw6_hip_synth_blocks(p, quant, bytes / (quant == Q6_K ? 210u : 144u), 0, SEED,
                                 stream_id(0, kind, e), NULL))
            return -1;
        mats[e].data = p;
        mats[e].quant = quant;
        mats[e].rows = rows;
        mats[e].cols = cols;
    }
    return 0;
}

static int make_matrix(qw6_hip_ctx_t *ctx, int quant, uint32_t kind, uint32_t rows, uint32_t cols,
                       qw6_hip_matrix_t *m) {
    const size_t bytes = matrix_bytes(quant, rows, cols);
    void *p = NULL;
    if (qw6_hip_alloc(ctx, bytes, &p)) return -1;
    if (qw6_hip_synth_blocks(p, quant, bytes / (quant == Q6_K ? 210u : 144u), 0, SEED,
                             stream_id(0, kind, 0), NULL))
        return -1;
    m->data = p;
    m->quant = quant;
    m->rows = rows;
    m->cols = cols;
    return 0;
}

/* one call's results against the golden answer */
static void compare(const char *what, const uint32_t *idx, const float *w, const float *out,
                    const int32_t *g_idx, const float *g_w, const float *g_out) {
    double num = 0.0, den = 0.0, wmax = 0.0;
    int idx_ok = 1;
    for (uint32_t k = 0; k < TOP_K; k++) {
        if ((int32_t)idx[k] != g_idx[k]) idx_ok = 0;
        const double d = fabs((double)w[k] - (double)g_w[k]);
        if (d > wmax) wmax = d;
    }
    for (uint32_t i = 0; i < HIDDEN; i++) {
        const double d = (double)out[i] - (double)g_out[i];
        num += d * d;
        den += (double)g_out[i] * (double)g_out[i];
    }
    const double rel = sqrt(num / (den > 0.0 ? den : 1e-300));
    const int ok = idx_ok && wmax <= 2e-5 && rel <= 1e-5;
    printf("%s: idx %s, max |dw| %.2e, rel-L2 %.2e -> %s\n", what, idx_ok ? "equal" : "DIFFER",
           wmax, rel, ok ? "ok" : "FAIL");
    if (!ok) fails++;
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s GOLDEN_DIR\n", argv[0]);
        return 2;
    }
    int32_t g_idx[TOP_K];
    float g_w[TOP_K];
    float *g_out = malloc(HIDDEN * sizeof(float));
    float *h_out = malloc(HIDDEN * sizeof(float));
    CHECK(g_out && h_out, "host allocation");
    CHECK(read_file(argv[1], "idx.bin", g_idx, sizeof g_idx) == 0 &&
              read_file(argv[1], "w.bin", g_w, sizeof g_w) == 0 &&
              read_file(argv[1], "out.bin", g_out, HIDDEN * sizeof(float)) == 0,
          "golden files in %s", argv[1]);

    /* 1. the Vulkan self-test's replacement and the F32 probe, by qw6's names */
    CHECK(qw6_vk_selftest() == 0, "qw6_vk_selftest");
    printf("selftest: ok\n");
    {
        enum { R = 7, C = 19 };
        float wf[R * C], xf[C], yf[R];
        for (int r = 0; r < R; r++)
            for (int c = 0; c < C; c++) wf[r * C + c] = 0.01f * (float)(r - c);
        for (int c = 0; c < C; c++) xf[c] = cosf(0.2f * (float)c);
        CHECK(qw6_vk_matvec_f32_host(wf, xf, yf, R, C) == 0, "qw6_vk_matvec_f32_host");
        double err = 0.0;
        for (int r = 0; r < R; r++) {
            double want = 0.0;
            for (int c = 0; c < C; c++) want += (double)wf[r * C + c] * (double)xf[c];
            const double d = fabs(want - (double)yf[r]);
            if (d > err) err = d;
        }
        printf("f32 host matvec 7x19: max err %.2e -> %s\n", err, err < 2e-5 ? "ok" : "FAIL");
        if (err >= 2e-5) fails++;
    }

    /* 2. the seeded layer, generated on the device */
    qw6_hip_ctx_t *ctx = NULL;
    CHECK(qw6_hip_ctx_init(&ctx, 0, 1) == 0, "qw6_hip_ctx_init");
    qw6_hip_matrix_t *gate = calloc(N_EXPERTS, sizeof *gate);
    qw6_hip_matrix_t *up = calloc(N_EXPERTS, sizeof *up);
    qw6_hip_matrix_t *down = calloc(N_EXPERTS, sizeof *down);
    CHECK(gate && up && down, "host allocation");
    CHECK(make_pack(ctx, Q4_K_M, K_GATE, INTER, HIDDEN, gate) == 0, "gate pack");
    CHECK(make_pack(ctx, Q4_K_M, K_UP, INTER, HIDDEN, up) == 0, "up pack");
    CHECK(make_pack(ctx, Q6_K, K_DOWN, HIDDEN, INTER, down) == 0, "down pack");
    qw6_hip_experts_t *experts = NULL;
    CHECK(qw6_hip_experts_create(ctx, gate, up, down, N_EXPERTS, &experts) == 0, "experts");
    void *router = NULL, *x = NULL, *out = NULL, *idx = NULL, *w = NULL;
    CHECK(qw6_hip_alloc(ctx, (size_t)N_EXPERTS * HIDDEN * sizeof(float), &router) == 0, "router");
    CHECK(qw6_hip_synth_normal(router, (uint64_t)N_EXPERTS * HIDDEN, 0.0f, 0.02f, SEED,
                               stream_id(0, K_ROUTER, 0), NULL) == 0, "router synth");
    qw6_hip_moe_layer_t L;
    memset(&L, 0, sizeof L);
    L.hidden = HIDDEN;
    L.inter = INTER;
    L.top_k = TOP_K;
    L.router = router;
    L.experts = experts;
    CHECK(make_matrix(ctx, Q4_K_M, K_SGATE, INTER, HIDDEN, &L.shared_gate) == 0 &&
              make_matrix(ctx, Q4_K_M, K_SUP, INTER, HIDDEN, &L.shared_up) == 0 &&
              make_matrix(ctx, Q6_K, K_SDOWN, HIDDEN, INTER, &L.shared_down) == 0,
          "shared expert");
    CHECK(qw6_hip_alloc(ctx, HIDDEN * sizeof(float), &x) == 0 &&
              qw6_hip_alloc(ctx, HIDDEN * sizeof(float), &out) == 0 &&
              qw6_hip_alloc(ctx, TOP_K * sizeof(uint32_t), &idx) == 0 &&
              qw6_hip_alloc(ctx, TOP_K * sizeof(float), &w) == 0,
          "activations");
    CHECK(qw6_hip_synth_normal(x, HIDDEN, 0.0f, 1.0f, SEED, stream_id(0, K_X, 0), NULL) == 0, "x");
    HIPCHECK(hipDeviceSynchronize());
    printf("layer: 256 experts generated on the device\n");

    /* 3. eager, then captured and replayed */
    hipStream_t s;
    HIPCHECK(hipStreamCreate(&s));
    uint32_t h_idx[TOP_K];
    float h_w[TOP_K];
    CHECK(qw6_hip_moe_forward(ctx, &L, x, NULL, NULL, 1, out, idx, w, s) == 0, "moe_forward");
    HIPCHECK(hipStreamSynchronize(s));
    HIPCHECK(hipMemcpy(h_out, out, HIDDEN * sizeof(float), hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(h_idx, idx, sizeof h_idx, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(h_w, w, sizeof h_w, hipMemcpyDeviceToHost));
    compare("eager", h_idx, h_w, h_out, g_idx, g_w, g_out);

    hipGraph_t graph;
    hipGraphExec_t exec;
    HIPCHECK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    const int rc = qw6_hip_moe_forward(ctx, &L, x, NULL, NULL, 1, out, idx, w, s);
    HIPCHECK(hipStreamEndCapture(s, &graph));
    CHECK(rc == 0, "moe_forward under capture");
    HIPCHECK(hipGraphInstantiate(&exec, graph, NULL, NULL, 0));
    for (int rep = 0; rep < 3; rep++) {
        HIPCHECK(hipMemsetAsync(out, 0, HIDDEN * sizeof(float), s));   /* outside the graph */
        HIPCHECK(hipMemsetAsync(idx, 0xff, TOP_K * sizeof(uint32_t), s));
        HIPCHECK(hipGraphLaunch(exec, s));
        HIPCHECK(hipStreamSynchronize(s));
        HIPCHECK(hipMemcpy(h_out, out, HIDDEN * sizeof(float), hipMemcpyDeviceToHost));
        HIPCHECK(hipMemcpy(h_idx, idx, sizeof h_idx, hipMemcpyDeviceToHost));
        HIPCHECK(hipMemcpy(h_w, w, sizeof h_w, hipMemcpyDeviceToHost));
        char what[32];
        snprintf(what, sizeof what, "graph replay %d", rep);
        compare(what, h_idx, h_w, h_out, g_idx, g_w, g_out);
    }
    HIPCHECK(hipGraphExecDestroy(exec));
    HIPCHECK(hipGraphDestroy(graph));
    HIPCHECK(hipStreamDestroy(s));

    qw6_hip_experts_free(experts);
    qw6_hip_ctx_free(ctx);
    free(gate);
    free(up);
    free(down);
    free(g_out);
    free(h_out);
    printf("%s\n", fails ? "FAIL" : "ok");
    return fails != 0;
}
