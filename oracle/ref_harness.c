/* ref_harness.c -- build-recipe helper for oracle/_ref (test infrastructure).
 *
 * Compiles qw6's own CPU path from the reference tree, unmodified, into a
 * shared library the tests can call: the reference's qw6.c is included as a
 * translation unit (its static dequant and MoE routines become reachable),
 * and these entry points wrap them behind plain pointers and sizes. Built by
 * oracle/Makefile only where the reference tree is present; the result lives
 * in oracle/_ref/ and is never linked by the product.
 */
#include "qw6.c"

static void ref_tensor(qw6_tensor_t *t, int quant, const void *data,
                       uint32_t rows, uint32_t cols) {
    memset(t, 0, sizeof *t);
    t->rows = rows;
    t->cols = cols;
    t->ne[0] = cols;
    t->ne[1] = rows;
    t->n_dims = 2;
    t->quant = (qw6_quant_t)quant;
    t->data = (void *)data;
}

float ref_fp16_to_f32(uint16_t h) { return qw6_fp16_to_f32(h); }

int ref_dequant_row(int quant, const void *data, uint32_t rows, uint32_t cols,
                    uint32_t row, float *dst) {
    qw6_tensor_t t;
    ref_tensor(&t, quant, data, rows, cols);
    return qw6_tensor_dequantize_row(&t, row, dst);
}

int ref_matvec(float *out, int quant, const void *data, uint32_t rows,
               uint32_t cols, const float *x, uint32_t max_rows) {
    qw6_tensor_t t;
    ref_tensor(&t, quant, data, rows, cols);
    return qw6_tensor_matvec(out, &t, x, max_rows);
}

void ref_moe_route(int *idx, float *w, const float *logits, int n, int k) {
    qw6_cpu_moe_route(idx, w, logits, n, k);
}

void ref_rmsnorm(float *out, const float *x, const float *w, int dim) {
    qw6_cpu_rmsnorm(out, x, w, dim);
}

/* One MoE layer through qw6_apply_layer_moe on a model whose layer 0 holds
 * the given tensors (router F32 [256 x 2048]; per-expert gate/up/down
 * pointers and quants; shared expert optional). Also returns the routing the
 * layer used (router matvec + qw6_cpu_moe_route, as the layer computes it). */
static int moe_layer_sr(float *out, int *idx, float *w, const float *router,
                        const void *const *gate, const int *gate_q,
                        const void *const *up, const int *up_q,
                        const void *const *down, const int *down_q,
                        const void *sgate, int sgate_q, const void *sup, int sup_q,
                        const void *sdown, int sdown_q, const float *x,
                        const float *shared_router) {
    qw6_model_t *m = calloc(1, sizeof *m);
    if (!m) return -1;
    ref_tensor(&m->layers[0].moe_router, QW6_Q_FP32, router, QW6_NUM_EXPERTS,
               QW6_HIDDEN_SIZE);
    if (shared_router)   /* F32 [1 x hidden]: weight sigmoid(w . x) */
        ref_tensor(&m->layers[0].shared_router, QW6_Q_FP32, shared_router, 1,
                   QW6_HIDDEN_SIZE);
    for (int e = 0; e < QW6_NUM_EXPERTS; e++) {
        ref_tensor(&m->layers[0].expert_gate[e], gate_q[e], gate[e], QW6_MOE_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&m->layers[0].expert_up[e], up_q[e], up[e], QW6_MOE_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&m->layers[0].expert_down[e], down_q[e], down[e], QW6_HIDDEN_SIZE, QW6_MOE_INTER);
    }
    if (sgate && sup && sdown) {
        ref_tensor(&m->layers[0].shared_gate, sgate_q, sgate, QW6_SHARED_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&m->layers[0].shared_up, sup_q, sup, QW6_SHARED_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&m->layers[0].shared_down, sdown_q, sdown, QW6_HIDDEN_SIZE, QW6_SHARED_INTER);
    }
    int rc = qw6_apply_layer_moe(out, m, 0, x);
    if (rc == 0 && idx && w) {
        float logits[QW6_NUM_EXPERTS];
        rc = qw6_tensor_matvec(logits, &m->layers[0].moe_router, x, QW6_NUM_EXPERTS);
        if (rc == 0)
            qw6_cpu_moe_route(idx, w, logits, QW6_NUM_EXPERTS, QW6_EXPERTS_PER_TOK);
    }
    free(m);
    return rc;
}

int ref_moe_layer(float *out, int *idx, float *w, const float *router,
                  const void *const *gate, const int *gate_q,
                  const void *const *up, const int *up_q,
                  const void *const *down, const int *down_q,
                  const void *sgate, int sgate_q, const void *sup, int sup_q,
                  const void *sdown, int sdown_q, const float *x) {
    return moe_layer_sr(out, idx, w, router, gate, gate_q, up, up_q, down, down_q,
                        sgate, sgate_q, sup, sup_q, sdown, sdown_q, x, NULL);
}

/* ref_moe_layer with the shared expert's gate sigmoid(shared_router . x)
 * (qw6.c:2267-2272). */
int ref_moe_layer_sr(float *out, int *idx, float *w, const float *router,
                     const void *const *gate, const int *gate_q,
                     const void *const *up, const int *up_q,
                     const void *const *down, const int *down_q,
                     const void *sgate, int sgate_q, const void *sup, int sup_q,
                     const void *sdown, int sdown_q, const float *x,
                     const float *shared_router) {
    return moe_layer_sr(out, idx, w, router, gate, gate_q, up, up_q, down, down_q,
                        sgate, sgate_q, sup, sup_q, sdown, sdown_q, x, shared_router);
}

/* The same MoE FFN with the router logits given (a batched-prefill token
 * whose logits come from elsewhere): qw6_apply_layer_moe's composition
 * (qw6.c:2248-2285) of the reference's own routines, minus the router
 * matvec; shared weight 1.0. */
int ref_moe_layer_logits(float *out, int *idx, float *w, const float *logits,
                         const void *const *gate, const int *gate_q,
                         const void *const *up, const int *up_q,
                         const void *const *down, const int *down_q,
                         const void *sgate, int sgate_q, const void *sup, int sup_q,
                         const void *sdown, int sdown_q, const float *x) {
    float g[QW6_MOE_INTER], u[QW6_MOE_INTER], mid[QW6_MOE_INTER];
    float tmp[QW6_HIDDEN_SIZE];
    qw6_tensor_t tg, tu, td;
    int rc = 0;
    memset(out, 0, QW6_HIDDEN_SIZE * sizeof(float));
    qw6_cpu_moe_route(idx, w, logits, QW6_NUM_EXPERTS, QW6_EXPERTS_PER_TOK);
    for (int k = 0; k < QW6_EXPERTS_PER_TOK && rc == 0; k++) {
        const int e = idx[k];
        ref_tensor(&tg, gate_q[e], gate[e], QW6_MOE_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&tu, up_q[e], up[e], QW6_MOE_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&td, down_q[e], down[e], QW6_HIDDEN_SIZE, QW6_MOE_INTER);
        rc = qw6_tensor_matvec(g, &tg, x, QW6_MOE_INTER);
        if (rc == 0) rc = qw6_tensor_matvec(u, &tu, x, QW6_MOE_INTER);
        if (rc == 0) {
            for (int i = 0; i < QW6_MOE_INTER; i++) mid[i] = qw6_silu(g[i]) * u[i];
            rc = qw6_tensor_matvec(tmp, &td, mid, QW6_HIDDEN_SIZE);
        }
        if (rc == 0)
            for (int i = 0; i < QW6_HIDDEN_SIZE; i++) out[i] += w[k] * tmp[i];
    }
    if (rc == 0 && sgate && sup && sdown) {
        const float sw = 1.0f;
        ref_tensor(&tg, sgate_q, sgate, QW6_SHARED_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&tu, sup_q, sup, QW6_SHARED_INTER, QW6_HIDDEN_SIZE);
        ref_tensor(&td, sdown_q, sdown, QW6_HIDDEN_SIZE, QW6_SHARED_INTER);
        rc = qw6_tensor_matvec(g, &tg, x, QW6_SHARED_INTER);
        if (rc == 0) rc = qw6_tensor_matvec(u, &tu, x, QW6_SHARED_INTER);
        if (rc == 0) {
            for (int i = 0; i < QW6_SHARED_INTER; i++) mid[i] = qw6_silu(g[i]) * u[i];
            rc = qw6_tensor_matvec(tmp, &td, mid, QW6_HIDDEN_SIZE);
        }
        if (rc == 0)
            for (int i = 0; i < QW6_HIDDEN_SIZE; i++) out[i] += sw * tmp[i];
    }
    return rc;
}

/* ---- qw6's GGUF reader (qw6.c:52-1240) on a file ---------------------------
 * Each call parses the file afresh with qw6_gguf_parse; -1 where qw6's own
 * call fails. */
static gguf_ctx_t *ref_gguf(const char *path) {
    gguf_ctx_t *c = calloc(1, sizeof *c);
    if (!c) return NULL;
    if (qw6_gguf_parse(path, c) != 0) {
        qw6_gguf_free(c);
        free(c);
        return NULL;
    }
    return c;
}

static void ref_gguf_done(gguf_ctx_t *c) {
    qw6_gguf_free(c);
    free(c);
}

int ref_gguf_header(const char *path, uint32_t *version, uint32_t *n_tensors,
                    uint32_t *n_kv, uint32_t *alignment, uint64_t *data_offset,
                    uint64_t *file_size) {
    gguf_ctx_t *c = ref_gguf(path);
    if (!c) return -1;
    *version = c->version;
    *n_tensors = c->tensors_parsed;
    *n_kv = c->kv_parsed;
    *alignment = c->alignment;
    *data_offset = c->data_offset;
    *file_size = c->file_size;
    ref_gguf_done(c);
    return 0;
}

/* qw6_gguf_parse followed by gguf_validate_tensor_ranges (as
 * qw6_gguf_read_file runs them, qw6.c:1100-1109). */
int ref_gguf_validate(const char *path) {
    gguf_ctx_t *c = ref_gguf(path);
    if (!c) return -1;
    int rc = gguf_validate_tensor_ranges(c);
    ref_gguf_done(c);
    return rc;
}

int ref_gguf_tensor(const char *path, uint32_t i, char *name, uint32_t *n_dims,
                    int64_t *dims, int32_t *type, uint64_t *offset,
                    uint64_t *span) {
    gguf_ctx_t *c = ref_gguf(path);
    if (!c) return -1;
    int rc = -1;
    if (i < c->tensors_parsed) {
        const gguf_tensor_info_t *ti = &c->tensors[i];
        memcpy(name, ti->name, sizeof ti->name);
        *n_dims = ti->n_dims;
        for (int d = 0; d < GGUF_MAX_DIMS; d++) dims[d] = ti->dims[d];
        *type = (int32_t)ti->type;
        *offset = ti->offset;
        *span = gguf_tensor_span(c, i, c->file_size);
        rc = 0;
    }
    ref_gguf_done(c);
    return rc;
}

/* bind_expert_pack on tensor i: every expert's file offset and size. */
int ref_gguf_pack(const char *path, uint32_t i, int32_t *quant, uint32_t *rows,
                  uint32_t *cols, uint64_t *offsets, uint64_t *sizes) {
    gguf_ctx_t *c = ref_gguf(path);
    if (!c) return -1;
    int rc = -1;
    qw6_tensor_t *dst = calloc(QW6_NUM_EXPERTS, sizeof *dst);
    if (dst && i < c->tensors_parsed) {
        const uint64_t abs = c->data_offset + c->tensors[i].offset;
        rc = bind_expert_pack(dst, &c->tensors[i], NULL, abs,
                              gguf_tensor_span(c, i, c->file_size));
        if (rc == 0) {
            *quant = (int32_t)dst[0].quant;
            *rows = dst[0].rows;
            *cols = dst[0].cols;
            for (int e = 0; e < QW6_NUM_EXPERTS; e++) {
                offsets[e] = dst[e].file_offset;
                sizes[e] = dst[e].data_size;
            }
        }
    }
    free(dst);
    ref_gguf_done(c);
    return rc;
}

/* qw6_gguf_find_kv: type, integer / float value, string. */
int ref_gguf_kv(const char *path, const char *key, int32_t *type, int64_t *ival,
                double *fval, char *str, size_t cap) {
    gguf_ctx_t *c = ref_gguf(path);
    if (!c) return -1;
    const gguf_kv_t *kv = qw6_gguf_find_kv(c, key);
    int rc = -1;
    if (kv) {
        *type = (int32_t)kv->type;
        *ival = 0;
        *fval = 0.0;
        switch (kv->type) {
            case GGUF_TYPE_UINT8: *ival = kv->val.u8; break;
            case GGUF_TYPE_INT8: *ival = kv->val.i8; break;
            case GGUF_TYPE_UINT16: *ival = kv->val.u16; break;
            case GGUF_TYPE_INT16: *ival = kv->val.i16; break;
            case GGUF_TYPE_UINT32: *ival = kv->val.u32; break;
            case GGUF_TYPE_INT32: *ival = kv->val.i32; break;
            case GGUF_TYPE_BOOL: *ival = kv->val.b; break;
            case GGUF_TYPE_UINT64: *ival = (int64_t)kv->val.u64; break;
            case GGUF_TYPE_INT64: *ival = kv->val.i64; break;
            case GGUF_TYPE_FLOAT32: *fval = kv->val.f32; break;
            case GGUF_TYPE_FLOAT64: *fval = kv->val.f64; break;
            default: break;
        }
        if (str && cap) {
            str[0] = 0;
            if (kv->type == GGUF_TYPE_STRING && kv->str)
                snprintf(str, cap, "%s", kv->str);
        }
        rc = 0;
    }
    ref_gguf_done(c);
    return rc;
}
