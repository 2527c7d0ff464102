/* qw6_oracle.h -- CPU restatement of qw6's routed-expert MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle: the parity tests,
 * the smoke check and the CPU-baseline leg of bench.py call it to compute the
 * expected result. Nothing in the product links it, and nothing here runs on
 * the GPU.
 *
 * It restates qw6.c's CPU reference (the correctness baseline of qw6) from
 * the GGUF block definitions, keeping the reference's fp32 evaluation order
 * so that, built with -std=c11 -O2 -ffp-contract=off, every output is
 * bit-identical to qw6.c's own. Each function names the reference lines it
 * follows. Bitwise equality with the reference is pinned by fixtures made
 * from the compiled reference (tests/golden) and by closed-form checks.
 *
 * Quant ids are qw6_quant_t values (qw6.h:76-91).
 */
#ifndef QW6_ORACLE_H
#define QW6_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_Q_FP32 = 0, ORC_Q_FP16 = 1, ORC_Q_BF16 = 2, ORC_Q_Q8_0 = 3,
    ORC_Q_Q4_K_M = 4, ORC_Q_Q4_K_S = 5, ORC_Q_Q5_K = 6, ORC_Q_Q6_K = 7,
    ORC_Q_Q3_K_M = 8, ORC_Q_IQ3_S = 9, ORC_Q_IQ3_XXS = 10, ORC_Q_IQ2_S = 11,
    ORC_Q_IQ2_M = 12, ORC_Q_IQ2_XXS = 13
};

/* One weight matrix in GGUF layout: rows x cols, row r at data + r*row_size. */
typedef struct {
    const void *data;
    int32_t quant;
    uint32_t rows;
    uint32_t cols;
} orc_mat_t;

float orc_fp16_to_f32(uint16_t h);
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m);
size_t orc_block_bytes(int quant);            /* 0 for non-block quants */
size_t orc_row_bytes(int quant, uint32_t cols); /* 0 if unsupported */

/* Expanded IQ lattice tables as the little-endian byte images the format
 * defines (for table checksums). */
void orc_iq_tables(uint64_t *iq2xxs, uint64_t *iq2s, uint32_t *iq3s,
                   uint8_t *ksigns, uint8_t *kmask);

int orc_dequant_row(int quant, const void *data, uint32_t cols, uint32_t row,
                    float *dst);
int orc_matvec(float *out, const orc_mat_t *w, const float *x,
               uint32_t max_rows, int nthreads);
void orc_moe_route(int *idx, float *weights, const float *logits,
                   int n_experts, int top_k);
void orc_rmsnorm(float *out, const float *x, const float *w, int dim,
                 float eps);
/* Greedy next token: the first index whose value is strictly greater than
 * every earlier one (qw6_cpu_argmax, qw6.c:2858-2863). n >= 1. */
int orc_argmax(const float *x, int n);
float orc_silu(float x);
float orc_sigmoid(float x);
void orc_silu_mul(const float *gate, const float *up, float *out, uint32_t n);
void orc_moe_gather(const float *expert_out, const float *expert_weights,
                    const float *shared_out, float shared_weight, float *out,
                    uint32_t dim, uint32_t top_k);

/* One MoE FFN for one token (qw6.c:2226-2290).
 * router: F32 [n_experts x hidden], or NULL when logits_in supplies the
 * router logits. experts: n_experts*3 matrices, [e*3+0]=gate, +1=up, +2=down.
 * shared: 3 matrices (gate, up, down) or NULL. shared_router: F32 [hidden] or
 * NULL (weight 1.0). idx_out/w_out: top_k selected experts and gate weights. */
int orc_moe_layer(float *out, int *idx_out, float *w_out,
                  const float *router, const float *logits_in,
                  const orc_mat_t *experts, const orc_mat_t *shared,
                  const float *shared_router, const float *x,
                  uint32_t hidden, uint32_t n_experts, uint32_t top_k,
                  int nthreads);

#ifdef __cplusplus
}
#endif
#endif
