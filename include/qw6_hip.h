/* qw6_hip.h -- C ABI of the MI355X (gfx950) routed-expert MoE FFN path.
 *
 * A drop-in for the matmul / MoE dispatch surface of qw6's Vulkan backend
 * (qw6_vk.h) on AMD Instinct MI355X: the same host operations with the same
 * argument meaning and 0 / -1 return codes, plus a device-resident API that
 * replaces the per-op pipeline dispatches of the MoE block
 * (qw6_vk.c:3350-3443) with three fused HIP kernels per layer.
 *
 * Conventions (kept from qw6_vk.h / qw6_vk.c):
 *  - every function returns 0 on success and -1 on failure, with a message on
 *    stderr; the library never exits the process;
 *  - weights are GGUF super-blocks of 256 columns, rows stored consecutively
 *    (row r at data + r * row_size), cols % 256 == 0;
 *  - quant ids are qw6_quant_t values (qw6.h:76-91): Q4_K_M=4, Q4_K_S=5,
 *    Q5_K=6, Q6_K=7, IQ3_S=9, IQ2_S=11, IQ2_XXS=13, FP32=0;
 *  - host ("_host") calls are synchronous and copy in / out of buffers they
 *    allocate per call, like qw6_vk.c:1186-1362;
 *  - device calls take device pointers and a hipStream_t passed as void*
 *    (NULL = the null stream) and are asynchronous on that stream.
 * Not thread-safe: one context per thread (qw6's pipe has the same rule,
 * qw6_vk.c:2154-2156).
 */
#ifndef QW6_HIP_H
#define QW6_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synchronous host operations (qw6_vk.h:9-56) ------------------------ */

/* y[rows] = W[rows x cols] x, F32 weights. Replaces qw6_vk_matvec_f32_host
 * (qw6_vk.h:10-11). */
int qw6_hip_matvec_f32_host(const float *w, const float *x, float *y,
                            uint32_t rows, uint32_t cols);
/* y = deq(W) x for one GGUF format. Replace qw6_vk_matmul_{q4k,q5k,q6k,
 * iq2xxs}_host (qw6_vk.h:12-19). The iq2s / iq3s variants have no host
 * wrapper in qw6 (those formats are pipe-only there, qw6_vk.c:2414-2425). */
int qw6_hip_matmul_q4k_host(const void *w, const float *x, float *y,
                            uint32_t rows, uint32_t cols);
int qw6_hip_matmul_q5k_host(const void *w, const float *x, float *y,
                            uint32_t rows, uint32_t cols);
int qw6_hip_matmul_q6k_host(const void *w, const float *x, float *y,
                            uint32_t rows, uint32_t cols);
int qw6_hip_matmul_iq2xxs_host(const void *w, const float *x, float *y,
                               uint32_t rows, uint32_t cols);
int qw6_hip_matmul_iq2s_host(const void *w, const float *x, float *y,
                             uint32_t rows, uint32_t cols);
int qw6_hip_matmul_iq3s_host(const void *w, const float *x, float *y,
                             uint32_t rows, uint32_t cols);
/* out = silu(gate) * up. Replaces qw6_vk_silu_mul_host (qw6_vk.h:24-25). */
int qw6_hip_silu_mul_host(const float *gate, const float *up, float *out,
                          uint32_t n);
/* Softmax top-k routing. Replaces qw6_vk_moe_route_host (qw6_vk.h:34-36):
 * n_experts <= 256, top_k <= 8; indices bit-exact with qw6_cpu_moe_route
 * (qw6.c:2796-2827) for the same logits. */
int qw6_hip_moe_route_host(const float *logits, uint32_t *indices,
                           float *weights, uint32_t n_experts, uint32_t top_k);
/* out[i] = sum_e w_e * expert_out[e][i] (+ shared_weight * shared_out[i]).
 * Replaces qw6_vk_moe_gather_host (qw6_vk.h:37-40); shared_out may be NULL. */
int qw6_hip_moe_gather_host(const float *expert_out,
                            const float *expert_weights,
                            const float *shared_out, float shared_weight,
                            float *out, uint32_t dim, uint32_t top_k);
/* y = x * (1 / sqrt(mean(x^2) + eps)) * w. Replaces qw6_vk_rmsnorm_host
 * (qw6_vk.h:20-21). */
int qw6_hip_rmsnorm_host(const float *x, const float *w, float *y, uint32_t n,
                         float eps);

/* ---- device-resident context (role of qw6_vk_pipe_t, qw6_vk.h:60-83) ---- */

typedef struct qw6_hip_ctx_s qw6_hip_ctx_t;

/* Create a context on HIP device `device`, with workspace for up to max_tokens
 * tokens per MoE call (decode: 1, MTP verify: 2, prefill: e.g. 512).
 * Mirrors qw6_vk_pipe_init (qw6_vk.h:63). */
int qw6_hip_ctx_init(qw6_hip_ctx_t **ctx, int device, uint32_t max_tokens);
/* Mirrors qw6_vk_pipe_free (qw6_vk.h:82). */
void qw6_hip_ctx_free(qw6_hip_ctx_t *ctx);

/* Copy `bytes` of host data into a new device buffer (256-B aligned) owned by
 * the context; *dev receives its address. Role of qw6_vk_upload_tensor
 * (qw6_vk.c:2366-2381), which records t->vk_offset. */
int qw6_hip_upload(qw6_hip_ctx_t *ctx, const void *host, size_t bytes,
                   void **dev);
/* A zeroed device buffer owned by the context. */
int qw6_hip_alloc(qw6_hip_ctx_t *ctx, size_t bytes, void **dev);

/* One weight matrix resident on the device. Takes explicit fields instead of
 * qw6_tensor_t* because that struct's layout depends on -DQW6_VULKAN
 * (qw6.h:105-107). */
typedef struct {
    const void *data;   /* device pointer, 16-byte aligned */
    int32_t quant;      /* qw6_quant_t */
    uint32_t rows;      /* output dim (ne[1]) */
    uint32_t cols;      /* input dim (ne[0]), multiple of 256 */
} qw6_hip_matrix_t;

/* y[t][rows] = deq(W) x[t][cols] for t < n_tok tokens (x, y row-major,
 * device pointers; x 16-byte aligned for a quantized W). Role of
 * qw6_vk_pipe_matvec (qw6_vk.c:2386-2430). */
int qw6_hip_matvec(qw6_hip_ctx_t *ctx, const qw6_hip_matrix_t *w,
                   const float *x, float *y, uint32_t n_tok, void *stream);

/* Per-layer expert table: n_experts entries of {gate, up, down}. Built once
 * from host descriptors (validated: supported quant, gate/up [inter x hidden],
 * down [hidden x inter]) into a device table the kernels index after
 * routing. Role of bind_expert_pack (qw6.c:542-597) plus the per-expert
 * tensors of qw6_model_t (qw6.h:155-165). Per-expert quants may differ. */
typedef struct qw6_hip_experts_s qw6_hip_experts_t;
int qw6_hip_experts_create(qw6_hip_ctx_t *ctx, const qw6_hip_matrix_t *gate,
                           const qw6_hip_matrix_t *up,
                           const qw6_hip_matrix_t *down, uint32_t n_experts,
                           qw6_hip_experts_t **out);
void qw6_hip_experts_free(qw6_hip_experts_t *e);

/* One MoE FFN layer (qw6_apply_layer_moe, qw6.c:2226-2290). */
typedef struct {
    uint32_t hidden;              /* model dim, multiple of 256 */
    uint32_t inter;               /* expert intermediate dim, multiple of 256 */
    uint32_t top_k;               /* <= 8 */
    const float *router;          /* F32 [n_experts x hidden], or NULL when
                                     router logits are passed in */
    const float *shared_router;   /* F32 [hidden] (weight sigmoid(w.x)) or
                                     NULL (weight 1.0) */
    const qw6_hip_experts_t *experts;
    qw6_hip_matrix_t shared_gate; /* shared expert; data == NULL: none */
    qw6_hip_matrix_t shared_up;
    qw6_hip_matrix_t shared_down;
    const float *norm_w;          /* F32 [hidden]: the layer input is first
                                     RMSNorm'd with this weight (the MoE
                                     block's post-attention norm,
                                     qw6_vk.c:3351-3354; qw6.c:2476-2478), or
                                     NULL: the input is used as given */
    float norm_eps;               /* RMSNorm epsilon (qw6.h QW6_RMS_EPS) */
} qw6_hip_moe_layer_t;

/* out[t] = MoE(x[t]) for n_tok tokens (device pointers, row-major [n_tok x
 * hidden]). logits: NULL to run the router matvec, else device F32
 * [n_tok x n_experts] router logits (batched prefill). idx/w: optional device
 * outputs [n_tok x top_k] of the routing. residual: optional device
 * [n_tok x hidden] added to the output (hidden = resid + ffn, qw6.c:2482).
 * x, out, residual and the layer's router, shared_router and norm_w are
 * 16-byte aligned (a call with another alignment fails). Tokens are processed
 * by the per-token kernels in launches of up to 16 tokens (decode, MTP
 * verification, small batches) or by the grouped bf16-MFMA kernels
 * (prefill); see qw6_hip_set_mode. */
int qw6_hip_moe_forward(qw6_hip_ctx_t *ctx, const qw6_hip_moe_layer_t *layer,
                        const float *x, const float *logits,
                        const float *residual, uint32_t n_tok, float *out,
                        uint32_t *idx, float *w, void *stream);

/* qw6_hip_moe_forward without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops). No counterpart in the reference. Same arguments, results and
 * per-token kernels (launches of up to 16 tokens, 4 in mode 3; never the
 * grouped kernels, so mode 2 is refused); the kernels' workspace (router
 * logits, selection tables, expert intermediates, MFMA operands) is a 4 MiB
 * static device array of the library instead of context allocations (every
 * shape the per-token kernels take, hidden and inter up to 2048, needs at
 * most 3.7 MB; a layer needing more would be refused with an error). Each device has one
 * such array, shared by every context and call on that device: calls that
 * overlap on one device race, so issue them on one stream (or otherwise
 * order them). */
int qw6_hip_moe_forward_noalloc(qw6_hip_ctx_t *ctx,
                                const qw6_hip_moe_layer_t *layer,
                                const float *x, const float *logits,
                                const float *residual, uint32_t n_tok,
                                float *out, uint32_t *idx, float *w,
                                void *stream);

/* Path selection for qw6_hip_moe_forward:
 * 0 = automatic (default): the fp32 per-token kernels for calls of up to 16
 *     tokens (15 when the layer holds IQ formats), the grouped MFMA kernels
 *     from 17 (16) tokens on (one launch per expert format present, so layers
 *     whose experts differ in format take them too);
 * 1 = always the fp32 per-token kernels (launches of up to 16 tokens);
 * 2 = always the grouped MFMA kernels;
 * 3 = always the small-batch MFMA per-token kernels (launches of up to 4
 *     tokens).
 * Returns -1 for another value. */
int qw6_hip_set_mode(qw6_hip_ctx_t *ctx, int mode);


/* Per-kernel timing of qw6_hip_moe_forward on its launch stream (eager calls
 * only, not under graph capture). max_calls > 0 starts recording for up to
 * that many calls, 0 stops. Each of the three decode kernels (router,
 * gate/up, down) is launched with start/stop events that the dispatch itself
 * timestamps (hipExtLaunchKernel), so the durations carry no extra queue
 * packets. qw6_hip_profile_read synchronizes and returns the summed elapsed
 * ms of [router, gate_up, down] over the recorded calls. */
int qw6_hip_profile(qw6_hip_ctx_t *ctx, uint32_t max_calls);
int qw6_hip_profile_read(qw6_hip_ctx_t *ctx, float ms[3], uint32_t *calls);

/* y = rmsnorm(x) * w per token (qw6_cpu_rmsnorm, qw6.c:2503-2513). */
int qw6_hip_rmsnorm(qw6_hip_ctx_t *ctx, const float *x, const float *w,
                    float *y, uint32_t n, uint32_t n_tok, float eps,
                    void *stream);

/* ---- output head: greedy next token ------------------------------------- */

/* Index of the maximum of x[0..n), n >= 1, bit-exact with qw6_cpu_argmax
 * (qw6.c:2858-2863): the first index whose value is strictly greater than
 * every earlier one (ties -> lowest index; NaNs never win; a NaN at index 0
 * gives 0). Device op, the role of qw6's argmax.comp dispatch
 * (qw6_vk_pipe_sample_greedy, qw6_vk.c:3467-3478): x and *out device
 * pointers, asynchronous on `stream`. Uses a 4 KB context workspace
 * allocated on first use. */
int qw6_hip_argmax(qw6_hip_ctx_t *ctx, const float *x, uint32_t n,
                   uint32_t *out, void *stream);
/* The same, synchronous, host buffers in and out: *out_idx the index and
 * *out_val (if out_val is not NULL) the element x[*out_idx]. Replaces
 * qw6_vk_argmax_host (qw6_vk.h:26-27, qw6_vk.c:811-833, 1258-1265). */
int qw6_hip_argmax_host(const float *x, uint32_t n, uint32_t *out_idx,
                        float *out_val);
/* Greedy token of host logits[0..n): the index qw6_hip_argmax_host returns.
 * Replaces qw6_vk_sampling_greedy_host (qw6_vk.h:28-29, qw6_vk.c:835-856,
 * 1267-1274); n == 0 fails as there. Ties and NaNs follow qw6_cpu_argmax
 * (qw6.c:2858-2863), the rule qw6's CPU greedy path applies; qw6's Vulkan
 * sampling.comp starts from -FLT_MAX and merges per-lane winners by lane, so
 * it can return a later index among exactly equal maxima. */
int qw6_hip_sampling_greedy_host(const float *logits, uint32_t n,
                                 uint32_t *token);

/* Greedy token of the output head (qw6_forward_token's tail, qw6.c:2490-2493,
 * then qw6_cpu_argmax; the GPU path of qw6_vk_pipe_forward_greedy,
 * qw6_vk.c:3447-3478): logits = deq(W) rmsnorm(x) * norm_w, *token =
 * argmax(logits). W: [vocab x hidden] (GGUF format or F32); norm_w NULL skips
 * the norm; x and norm_w 16-byte aligned; logits: device buffer of W->rows
 * floats (written, as qw6's scr_logits); token: one device uint32.
 * Asynchronous on `stream`. */
int qw6_hip_output_greedy(qw6_hip_ctx_t *ctx, const qw6_hip_matrix_t *w,
                          const float *x, const float *norm_w, float eps,
                          float *logits, uint32_t *token, void *stream);

/* ---- seeded synthetic data on the device -------------------------------- */

/* Fill `nblocks` GGUF blocks of format `quant` from (seed, stream), starting
 * at block `first`: the device twin of qw6_amd/synth.py quant_blocks. */
int qw6_hip_synth_blocks(void *dst, int32_t quant, uint64_t nblocks,
                         uint64_t first, uint64_t seed, uint64_t stream_id,
                         void *stream);
/* n floats mean + std * z (z: the generator's standard normal deviates). */
int qw6_hip_synth_normal(float *dst, uint64_t n, float mean, float std,
                         uint64_t seed, uint64_t stream_id, void *stream);

/* Device self-test: known-answer inputs (unit-scale K-quant blocks with
 * patterned codes, zero-index IQ blocks, a dense F32 matrix, SiLU*up, a tied
 * routing case, the weighted gather) through the host operations above,
 * checked against closed forms; one line per case on stderr. 0 when every
 * case passes. Replaces qw6_vk_selftest (qw6_vk.h:9, qw6_vk.c:1514-2133). */
int qw6_hip_selftest(void);

/* Last error message of the calling thread ("" if none). */
const char *qw6_hip_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
