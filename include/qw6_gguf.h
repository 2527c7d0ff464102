/* qw6_gguf.h -- GGUF v3 weight residency for the MI355X MoE FFN path.
 *
 * Parses a GGUF model file the way qw6's loader does (qw6.c:52-1240), binds
 * the MoE tensors of a layer with qw6's expert-pack rule (bind_expert_pack,
 * qw6.c:542-597) and streams them from the file into device memory through
 * pinned staging buffers -- the role of qw6_vk_upload_tensor
 * (qw6_vk.c:2366-2381) in qw6_vk_pipe_init's upload loop
 * (qw6_vk.c:2926-2958). The on-disk expert packs are the on-device format:
 * the kernels read the GGUF blocks as they are in the file.
 *
 * Conventions of qw6_hip.h apply: 0 / -1 returns, the message on stderr and
 * in qw6_hip_last_error(); device buffers made here are owned by the context
 * and freed by qw6_hip_ctx_free. A qw6_hip_gguf_t is read-only after
 * qw6_hip_gguf_open and may be shared by contexts on several devices, but
 * its staging buffers are not thread-safe: upload from one thread at a time.
 */
#ifndef QW6_GGUF_H
#define QW6_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "qw6_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qw6_hip_gguf_s qw6_hip_gguf_t;

/* Open and parse a GGUF v3 file: header, metadata key/value pairs and tensor
 * table (qw6_gguf_parse, qw6.c:871-1075), with qw6's limits (<= 512 pairs,
 * <= 4096 tensors, <= 4 dims, strings <= 1 MiB, arrays <= 10 Mi elements,
 * names and keys kept to 127 bytes). The data section starts at the end of
 * the table rounded up to general.alignment (a UINT32 key; default 32). Every
 * tensor's byte range is then checked against the file size with qw6's
 * per-type block sizes (gguf_validate_tensor_ranges, qw6.c:410-457): a tensor
 * of a type outside F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_S,
 * IQ3_S, or a truncated file, fails the open. */
int qw6_hip_gguf_open(const char *path, qw6_hip_gguf_t **out);
void qw6_hip_gguf_close(qw6_hip_gguf_t *g);

/* Header facts (gguf_ctx_t fields, qw6.h:420-431); any pointer may be NULL. */
int qw6_hip_gguf_header(const qw6_hip_gguf_t *g, uint32_t *version,
                        uint32_t *n_tensors, uint32_t *n_kv,
                        uint32_t *alignment, uint64_t *data_offset,
                        uint64_t *file_size);

/* Tensor i of the table (gguf_tensor_info_t, qw6.h:411-417): name (NUL-
 * terminated, at most 127 bytes, into name[128]), dims, ggml type, offset
 * relative to the data section, and its span -- the bytes up to the next
 * tensor's start or the end of the file (gguf_tensor_span, qw6.c:459-470).
 * Any output pointer may be NULL. */
int qw6_hip_gguf_tensor(const qw6_hip_gguf_t *g, uint32_t i, char *name,
                        uint32_t *n_dims, int64_t dims[4], int32_t *ggml_type,
                        uint64_t *offset, uint64_t *span);
/* Index of the first tensor named `name`, or -1 (no message). */
int qw6_hip_gguf_find_tensor(const qw6_hip_gguf_t *g, const char *name);

/* Metadata lookup by key (qw6_gguf_find_kv, qw6.c:271-279): the first pair
 * with that key. _kv_type gives its gguf_type_t (-1: absent); _kv_int the
 * value of an integer or BOOL scalar; _kv_float of a FLOAT32 / FLOAT64
 * scalar; _kv_str copies a STRING (truncated to cap - 1 bytes, NUL-
 * terminated). The typed getters return -1 for a missing key or another
 * type. */
int32_t qw6_hip_gguf_kv_type(const qw6_hip_gguf_t *g, const char *key);
int qw6_hip_gguf_kv_int(const qw6_hip_gguf_t *g, const char *key,
                        int64_t *val);
int qw6_hip_gguf_kv_float(const qw6_hip_gguf_t *g, const char *key,
                          double *val);
int qw6_hip_gguf_kv_str(const qw6_hip_gguf_t *g, const char *key, char *buf,
                        size_t cap);

/* The expert-pack rule of bind_expert_pack (qw6.c:542-597) for tensor i: a
 * 3-dim tensor [cols, rows, n_experts] (n_experts == 0: qw6's 256) of a type
 * qw6 maps to a qw6_quant_t (qw6_gguf_to_quant, qw6.c:1079-1094), whose
 * n_experts * rows * row_size bytes fit in the tensor's span. Expert e's
 * rows start at file offset *file_offset + e * *expert_bytes. */
int qw6_hip_gguf_expert_pack(const qw6_hip_gguf_t *g, uint32_t i,
                             uint32_t n_experts, int32_t *quant,
                             uint32_t *rows, uint32_t *cols,
                             uint64_t *file_offset, uint64_t *expert_bytes);

/* Copy tensor i into a new device buffer (256-B aligned, owned by ctx),
 * streaming the file through pinned staging buffers. *out gets its address,
 * qw6_quant_t, rows (the product of dims[1..]) and cols (dims[0]). Role of
 * qw6_tensor_bind (qw6.c:483-508) followed by qw6_vk_upload_tensor
 * (qw6_vk.c:2366-2381). */
int qw6_hip_gguf_upload(qw6_hip_ctx_t *ctx, qw6_hip_gguf_t *g, uint32_t i,
                        qw6_hip_matrix_t *out);

/* The MoE block of layer `layer` made resident and described for
 * qw6_hip_moe_forward. Tensors of blk.<layer>. (bind_layer_tensor,
 * qw6.c:599-677):
 *   ffn_gate_inp.weight       router, F32 [hidden, n_experts]   (required)
 *   ffn_{gate,up}_exps.weight expert packs [hidden, inter, n_experts]
 *   ffn_down_exps.weight      expert pack  [inter, hidden, n_experts]
 *                                                              (required)
 *   ffn_{gate,up,down}_shexp.weight  shared expert   (all three or none)
 *   ffn_gate_inp_shexp.weight shared-expert gate, F32 [hidden]  (optional;
 *                             used with the shared expert only)
 *   post_attention_norm.weight  RMSNorm weight, F32 [hidden]    (optional)
 * top_k is <arch>.expert_count_used when present (else 8), the RMSNorm
 * epsilon <arch>.attention.layer_norm_rms_epsilon (else 1e-6), <arch> being
 * general.architecture. Missing required tensors are named in the error, as
 * in qw6_validate_layer_bindings (qw6.c:679-798). desc->norm_w is set when
 * the norm weight is present; clear it to pass the input through as given.
 * *experts is the layer's expert table (free with qw6_hip_experts_free);
 * every device buffer belongs to ctx. */
int qw6_hip_gguf_moe_layer(qw6_hip_ctx_t *ctx, qw6_hip_gguf_t *g,
                           uint32_t layer, qw6_hip_moe_layer_t *desc,
                           qw6_hip_experts_t **experts);

#ifdef __cplusplus
}
#endif
#endif
