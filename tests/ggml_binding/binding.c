/*
 * binding.c — the ggml-side binding of the attention path, as a maintainer
 * adds it to a ggml GPU backend (its supports_op and graph_compute hooks),
 * compiled here as C against ggml_min.h and driven by
 * tests/test_gpu_ggml_binding.py through the nodes voxtral.cpp's decoder
 * builds (src/voxtral.cpp:1772-1802).
 *
 * Part 1 (vxfa_desc .. backend_flash_attn_ext) is the binding itself, the
 * text the integration guide shows. Part 2 is the test driver: it builds
 * each GGML_OP_FLASH_ATTN_EXT node the way ggml_view_2d, ggml_reshape_3d,
 * ggml_permute, ggml_cast and ggml_flash_attn_ext would (ne, nb, data,
 * op_params, src[]) and hands it to part 1.
 */
#include <math.h>
#include <stdbool.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "ggml_min.h"
#include "vxfa.h"

/* ---- part 1: the binding ------------------------------------------------- */

static vxfa_tensor vxfa_desc(const struct ggml_tensor * t) {
    vxfa_tensor d = {0};
    d.data = t->data;                 /* device pointer of the backend buffer            */
    d.type = (int32_t) t->type;       /* GGML_TYPE_F32 = 0, GGML_TYPE_F16 = 1: same codes */
    for (int i = 0; i < 4; ++i) { d.ne[i] = t->ne[i]; d.nb[i] = t->nb[i]; }
    return d;
}

/* op params of GGML_OP_FLASH_ATTN_EXT: scale, max_bias, logit_softcap (floats 0..2) */
static void vxfa_params(const struct ggml_tensor * node, float * scale, float * max_bias, float * softcap) {
    memcpy(scale,    (const float *) node->op_params + 0, sizeof(float));
    memcpy(max_bias, (const float *) node->op_params + 1, sizeof(float));
    memcpy(softcap,  (const float *) node->op_params + 2, sizeof(float));
}

/* supports_op: the scheduler falls back to the next backend (CPU last) on false */
static bool backend_supports_flash_attn_ext(const struct ggml_tensor * node) {
    const struct ggml_tensor * q = node->src[0], * k = node->src[1], * v = node->src[2], * m = node->src[3];
    if (node->src[4] != NULL) return false;                 /* attention sinks: not implemented */
    vxfa_tensor dq = vxfa_desc(q), dk = vxfa_desc(k), dv = vxfa_desc(v), dd = vxfa_desc(node), dm;
    if (m) dm = vxfa_desc(m);
    float scale, max_bias, softcap;
    vxfa_params(node, &scale, &max_bias, &softcap);
    return vxfa_supports(&dq, &dk, &dv, m ? &dm : NULL, &dd, scale, max_bias, softcap) == VXFA_OK;
}

/* graph_compute: one call per node, asynchronous on the backend's stream */
static bool backend_flash_attn_ext(vxfa_ctx * vctx, hipStream_t stream, struct ggml_tensor * node) {
    const struct ggml_tensor * q = node->src[0], * k = node->src[1], * v = node->src[2], * m = node->src[3];
    vxfa_tensor dq = vxfa_desc(q), dk = vxfa_desc(k), dv = vxfa_desc(v), dd = vxfa_desc(node), dm;
    if (m) dm = vxfa_desc(m);
    float scale, max_bias, softcap;
    vxfa_params(node, &scale, &max_bias, &softcap);
    const int rc = vxfa_flash_attn_ext(vctx, &dq, &dk, &dv, m ? &dm : NULL, &dd,
                                       scale, max_bias, softcap, (void *) stream);
    if (rc != VXFA_OK) {
        GGML_LOG_ERROR("vxfa: %s (%s)\n", vxfa_status_str(rc), vxfa_last_error(vctx));
        return false;
    }
    return true;
}

/* ---- part 2: test driver ------------------------------------------------- */

/* A contiguous tensor of ggml_new_tensor_4d. */
static struct ggml_tensor t_new(enum ggml_type type, void * data, int64_t ne0, int64_t ne1, int64_t ne2,
                                int64_t ne3) {
    struct ggml_tensor t;
    memset(&t, 0, sizeof(t));
    t.type = type;
    t.data = data;
    t.ne[0] = ne0; t.ne[1] = ne1; t.ne[2] = ne2; t.ne[3] = ne3;
    t.nb[0] = type == GGML_TYPE_F32 ? 4 : 2;
    for (int i = 1; i < 4; ++i) t.nb[i] = t.nb[i - 1] * (size_t) t.ne[i - 1];
    return t;
}

/* ggml_reshape_3d of a contiguous tensor to [ne0, ne1, ne2], then
 * ggml_permute(t, 0, 2, 1, 3), which swaps axes 1 and 2. */
static struct ggml_tensor t_reshape3_permute0213(const struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2) {
    struct ggml_tensor r = t_new(a->type, a->data, ne0, ne1, ne2, 1);
    const int64_t ne = r.ne[1];
    const size_t nb = r.nb[1];
    r.ne[1] = r.ne[2]; r.nb[1] = r.nb[2];
    r.ne[2] = ne;      r.nb[2] = nb;
    return r;
}

/* One decoder attention node of voxtral.cpp (src/voxtral.cpp:1772-1802):
 *   q        F32 [n_heads * head_dim, n_tokens] (contiguous, as after ggml_cont)
 *   k_cache  F32 kv_self_k [kv_dim, window, n_layers] (src/voxtral.cpp:1126-1136),
 *            likewise v_cache; the node reads layer `layer`, rows [0, n_kv)
 *   mask     F16 [n_kv, n_tokens] (the ggml_cast of the causal mask) or NULL
 *   dst      F32 [head_dim, n_heads, n_tokens]
 * sinks != 0 sets src[4] (an attention-sinks tensor) to exercise supports_op.
 * Returns 1 when supports_op accepts the node and graph_compute succeeds,
 * 0 when supports_op declines it, -1 when graph_compute fails. */
int vxfa_test_decoder_node(vxfa_ctx * vctx, void * stream, float * q, float * k_cache, float * v_cache,
                           int n_layers, int window, int layer, int n_heads, int n_kv_heads, int head_dim,
                           int n_tokens, int n_kv, void * mask, float * dst, int sinks) {
    const int64_t kv_dim = (int64_t) n_kv_heads * head_dim;
    (void) n_layers;

    struct ggml_tensor q2 = t_new(GGML_TYPE_F32, q, (int64_t) n_heads * head_dim, n_tokens, 1, 1);
    struct ggml_tensor q3 = t_reshape3_permute0213(&q2, head_dim, n_heads, n_tokens);

    /* ggml_view_2d(kv_self, kv_dim, n_kv, kv_self->nb[1], layer * kv_self->nb[2]) */
    const size_t cache_nb1 = (size_t) kv_dim * sizeof(float);
    const size_t cache_nb2 = cache_nb1 * (size_t) window;
    struct ggml_tensor k_full = t_new(GGML_TYPE_F32, (char *) k_cache + (size_t) layer * cache_nb2, kv_dim, n_kv, 1, 1);
    struct ggml_tensor v_full = t_new(GGML_TYPE_F32, (char *) v_cache + (size_t) layer * cache_nb2, kv_dim, n_kv, 1, 1);
    struct ggml_tensor k3 = t_reshape3_permute0213(&k_full, head_dim, n_kv_heads, n_kv);
    struct ggml_tensor v3 = t_reshape3_permute0213(&v_full, head_dim, n_kv_heads, n_kv);

    struct ggml_tensor m16 = t_new(GGML_TYPE_F16, mask, n_kv, n_tokens, 1, 1);
    struct ggml_tensor sink = t_new(GGML_TYPE_F32, NULL, n_heads, 1, 1, 1);

    /* ggml_flash_attn_ext(ctx, q3, k3, v3, mask, scale, 0.0f, 0.0f) */
    struct ggml_tensor node = t_new(GGML_TYPE_F32, dst, head_dim, n_heads, n_tokens, 1);
    node.op = GGML_OP_FLASH_ATTN_EXT;
    const float params[3] = {1.0f / sqrtf((float) head_dim), 0.0f, 0.0f};
    memcpy(node.op_params, params, sizeof(params));
    node.src[0] = &q3;
    node.src[1] = &k3;
    node.src[2] = &v3;
    node.src[3] = mask ? &m16 : NULL;
    node.src[4] = sinks ? &sink : NULL;

    if (!backend_supports_flash_attn_ext(&node)) return 0;
    return backend_flash_attn_ext(vctx, (hipStream_t) stream, &node) ? 1 : -1;
}
