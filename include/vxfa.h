/*
 * vxfa.h — C ABI of the MI355X (gfx950) attention path for voxtral.cpp.
 *
 * One operation: GGML_OP_FLASH_ATTN_EXT, with ggml's tensor contract.
 *
 *   dst = softmax(scale * Q K^T + mask) V, per query head, GQA-broadcast K/V.
 *
 * voxtral.cpp emits this op at two sites:
 *   src/voxtral.cpp:1611  encoder self-attention   (hd 64, no mask offline)
 *   src/voxtral.cpp:1802  decoder GQA attention    (32 q / 8 kv heads, hd 128,
 *                                                  causal mask or none)
 * Both pass max_bias = 0 and logit_softcap = 0.
 * The op constructor is ggml_flash_attn_ext(ctx, q, k, v, mask, scale,
 * max_bias, logit_softcap). It lives in ggml (external, pinned in
 * CMakeLists.txt:36-39). It is executed by a ggml backend's graph_compute,
 * which the scheduler calls from src/voxtral.cpp:2097, 2193, 2382.
 *
 * Tensor contract (ggml order, ne[0] fastest, nb in bytes):
 *   q    [D,  Nq,  Hq,  B ]  F32 or F16, rows contiguous (nb[0] = elt size)
 *   k    [D,  Nkv, Hkv, Bk]  F16 or F32, rows contiguous
 *   v    [D,  Nkv, Hkv, Bk]  same type as k, rows contiguous (not transposed)
 *   mask [Nkv, >=Nq, Hm, Bm] F16 additive (0 / -inf in voxtral), nullable,
 *                            elements contiguous along ne[0]
 *   dst  [D,  Hq,  Nq,  B ]  F32, contiguous (permuted relative to q)
 * with Hq % Hkv == 0, B % Bk == 0, Hq % Hm == 0, B % Bm == 0.
 * Query head h reads kv head h / (Hq / Hkv) and mask plane h % Hm.
 *
 * Semantics follow ggml's CPU kernel: a mask entry of -inf removes that kv
 * position; a query row with every position removed produces zeros.
 *
 * Everything here is plain C: pointers, sizes and status codes. No HIP or
 * torch types cross the boundary. The stream argument is a hipStream_t
 * passed as void* (NULL = the null stream).
 */
#ifndef VXFA_H
#define VXFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. The numeric values equal ggml's GGML_TYPE_F32 / GGML_TYPE_F16,
 * so a ggml backend can pass tensor->type through unchanged. */
enum vxfa_type {
    VXFA_TYPE_F32 = 0,
    VXFA_TYPE_F16 = 1,
};

/* Status codes. Nothing aborts and no C++ exception crosses the ABI.
 * VXFA_UNSUPPORTED plays the role of ggml's supports_op() == false: the
 * caller runs the op elsewhere (ggml's scheduler falls back to the CPU
 * backend, which voxtral lists last at src/voxtral.cpp:1167-1170). */
enum vxfa_status {
    VXFA_OK           = 0,
    VXFA_UNSUPPORTED  = 1,  /* valid op, but this path does not implement it  */
    VXFA_INVALID_ARG  = 2,  /* violates the ggml contract (shapes, strides)   */
    VXFA_NO_WORKSPACE = 3,  /* the context's fixed workspace is too small     */
    VXFA_HIP_ERROR    = 4,  /* a HIP call failed; see vxfa_last_error()       */
};

/* A ggml tensor view: exactly the fields of struct ggml_tensor that the op
 * reads (type, ne, nb, data). data is a device pointer. */
typedef struct vxfa_tensor {
    void*   data;
    int32_t type;   /* enum vxfa_type */
    int32_t pad_;   /* keep ne[] 8-byte aligned; ignored */
    int64_t ne[4];
    size_t  nb[4];
} vxfa_tensor;

/* Per-stream context (the analogue of a ggml backend context). Owns one
 * device workspace of fixed size, allocated by vxfa_ctx_create and freed by
 * vxfa_ctx_destroy: the split-KV partial records (8 MiB: partial O,
 * running max and sum per split) and an f16 staging
 * area for F32 K/V of prefill calls (32 MiB: K and V of up to 8192 rows of
 * 8 x 128). No other call allocates, frees or synchronises, so every call
 * can be captured into a HIP graph; a decode call whose batch would need more
 * partial records than the workspace holds runs with fewer splits, a prefill
 * call with F32 K/V beyond the staging area returns VXFA_NO_WORKSPACE. The
 * caller's tensors are never allocated or freed here. One context per
 * stream; calls on one context must not overlap. */
typedef struct vxfa_ctx vxfa_ctx;

/* Create a context bound to HIP device `device` and allocate its workspace
 * (40 MiB). Returns NULL on failure. */
vxfa_ctx* vxfa_ctx_create(int device);

/* Destroy a context and free its workspace. NULL is accepted. */
void vxfa_ctx_destroy(vxfa_ctx* ctx);

/* Capability check. Mirrors a ggml backend's supports_op() for
 * GGML_OP_FLASH_ATTN_EXT (the scheduler consults it when placing the node;
 * placement order is set at src/voxtral.cpp:1156-1175). Pure host code: it
 * only reads the descriptors, never dereferences data, and makes no HIP call,
 * so it runs on a machine without a GPU.
 * Returns VXFA_OK, VXFA_UNSUPPORTED or VXFA_INVALID_ARG. */
int vxfa_supports(const vxfa_tensor* q, const vxfa_tensor* k,
                  const vxfa_tensor* v, const vxfa_tensor* mask,
                  const vxfa_tensor* dst, float scale, float max_bias,
                  float logit_softcap);

/* Execute GGML_OP_FLASH_ATTN_EXT. Replaces the backend kernel behind
 * ggml_flash_attn_ext(ctx, q, k, v, mask, scale, max_bias, logit_softcap)
 * at src/voxtral.cpp:1611 and :1802. Asynchronous on `stream`: the call
 * returns after the launches are queued, with no host synchronisation and no
 * allocation. Output is deterministic for equal inputs (fixed split
 * boundaries and merge order). F32 K/V (the reference's own cache,
 * src/voxtral.cpp:1126-1136, and the encoder's K/V, :1581-1605): a decode
 * step reads them in place and keeps both products in F32 with Q unrounded,
 * as ggml's CPU kernel does for F32 K; a prefill call copies them to f16 in
 * the context's staging area first and rounds Q, K and V to f16 as for f16
 * K/V. */
int vxfa_flash_attn_ext(vxfa_ctx* ctx, const vxfa_tensor* q,
                        const vxfa_tensor* k, const vxfa_tensor* v,
                        const vxfa_tensor* mask, vxfa_tensor* dst, float scale,
                        float max_bias, float logit_softcap, void* stream);

/* Implicit masks. voxtral.cpp fills every mask it passes from a formula:
 *   decoder prefill   causal [n, n]           fill_causal_mask,
 *                                             src/voxtral.cpp:2104-2111
 *                                             (used at :2421 and :2493)
 *   realtime encoder  causal window of 750    src/voxtral.cpp:2179-2190
 * then uploads it and casts it to F16 inside every layer's graph (:1564,
 * :1801). A descriptor of the formula replaces the tensor: query row i
 * (0-based along q's ne[1]) attends kv position j iff
 *   j <= i + offset   and, when window > 0,   j >= i + offset - window + 1.
 * (Decoder prefill: offset 0, window 0. Realtime encoder: offset 0, window
 * 750. A decode step with a sliding window W over n_kv cached rows:
 * offset n_kv - 1, window W.) The result equals vxfa_flash_attn_ext with an
 * F16 mask [Nkv, Nq, 1, 1] holding 0 at those positions and -inf elsewhere.
 * The kernels derive live ranges and tile classes from the formula instead
 * of reading a mask, so no mask is filled, copied or scanned. */
enum vxfa_mask_kind {
    VXFA_MASK_NONE   = 0,  /* no mask: same as passing mask = NULL */
    VXFA_MASK_CAUSAL = 1,  /* causal, optionally limited to a window */
};

typedef struct vxfa_mask_desc {
    int32_t kind;    /* enum vxfa_mask_kind                                  */
    int32_t window;  /* 0: unbounded; W > 0: the last W positions up to the
                        diagonal                                             */
    int64_t offset;  /* kv position on query row 0's diagonal                 */
} vxfa_mask_desc;

/* Validate a mask descriptor (pure host code). NULL is valid (no mask).
 * Returns VXFA_OK or VXFA_INVALID_ARG. */
int vxfa_check_mask_desc(const vxfa_mask_desc* mask);

/* GGML_OP_FLASH_ATTN_EXT with an implicit mask (see above) in place of the
 * mask tensor; otherwise the same contract, status codes and stream
 * behaviour as vxfa_flash_attn_ext. No counterpart in ggml's op: it is for a
 * caller that owns the mask's formula (voxtral.cpp's builders at
 * src/voxtral.cpp:1801 and :1564 would pass a descriptor instead of the
 * cast mask tensor). mask = NULL or kind VXFA_MASK_NONE means no mask. */
int vxfa_flash_attn_ext_implicit(vxfa_ctx* ctx, const vxfa_tensor* q,
                                 const vxfa_tensor* k, const vxfa_tensor* v,
                                 const vxfa_mask_desc* mask, vxfa_tensor* dst,
                                 float scale, float max_bias,
                                 float logit_softcap, void* stream);

/* F16 KV cache append. build_decoder_layer stores each layer's new keys and
 * values with two ggml_cpy nodes into cache views (src/voxtral.cpp:1758-1770);
 * with an F16 cache these are F32 -> F16 conversions (round to nearest even,
 * overflow to inf). k_new, v_new: F32 [Hkv * D, n_new, 1, Bk], rows
 * contiguous (kv head h at elements h * D .. h * D + D - 1, the layout of
 * the reshape at :1743); k, v: the F16 cache views [D, n_kv, Hkv, Bk] the
 * attention op reads (:1773-1794). Rows n_kv - n_new .. n_kv - 1 of k and v
 * receive the new rows (voxtral's n_kv = kv_offset + n_tokens).
 * One launch for K and V; asynchronous on `stream`. */
int vxfa_kv_append(vxfa_ctx* ctx, const vxfa_tensor* k_new,
                   const vxfa_tensor* v_new, vxfa_tensor* k, vxfa_tensor* v,
                   void* stream);

/* vxfa_kv_append(k_new, v_new, k, v) followed by vxfa_flash_attn_ext(q, k,
 * v, mask, dst, ...), with the same result bits. For a single-token decode
 * step (Nq = 1, n_new = 1) the append is fused into the attention kernel:
 * the new row is read once from the F32 source, used, and written to the
 * cache by the same launch; otherwise the append kernel runs first on the
 * same stream. No counterpart in ggml's op: it replaces the two ggml_cpy
 * nodes plus the attention node of each decoder layer (:1758-1802). */
int vxfa_flash_attn_ext_append(vxfa_ctx* ctx, const vxfa_tensor* q,
                               vxfa_tensor* k, vxfa_tensor* v,
                               const vxfa_tensor* k_new,
                               const vxfa_tensor* v_new,
                               const vxfa_tensor* mask, vxfa_tensor* dst,
                               float scale, float max_bias,
                               float logit_softcap, void* stream);

/* KV cache as a ring buffer. Once its cache holds VOXTRAL_DEC_WINDOW rows,
 * voxtral.cpp moves every layer's K and V one row to the left before each
 * decode step (kv_cache_shift_left, src/voxtral.cpp:1237-1266, called at
 * :2446-2449): (window - 1) rows per layer, K and V, on every token. With a
 * ring the same step is O(1): logical position p (0 = oldest kept token)
 * lives in cache row (start + p) mod capacity, so dropping the oldest row is
 * start = (start + 1) mod capacity, and no row is moved or cleared (rows at
 * logical positions >= n_kv are never read, which also makes the full-cache
 * memset of clear_kv_cache, :1222-1235, unnecessary). */
typedef struct vxfa_ring {
    int64_t start;  /* cache row of logical position 0; 0 <= start < capacity */
    int64_t n_kv;   /* rows in use (logical 0 .. n_kv - 1); <= capacity        */
} vxfa_ring;

/* A decode step over a ring: q [D, 1, Hq, B]; k, v the whole cache
 * [D, capacity, Hkv, Bk] (F16); attention over logical positions
 * 0 .. n_kv - 1 with no mask (voxtral's decode steps pass none, :1961,
 * :2052). With k_new / v_new (F32 [Hkv * D, 1, 1, Bk], or both NULL) the
 * step's new row is logical position n_kv - 1: it is rounded to f16, used
 * and written to its ring row in the same launch (as
 * vxfa_flash_attn_ext_append). The result equals vxfa_flash_attn_ext on a
 * linear cache holding the same rows in logical order. Single-token decode
 * with GQA group 1, 2 or 4 only, capacity below 2^24 rows and capacity *
 * row stride below 2 GiB (else VXFA_UNSUPPORTED). No counterpart in
 * ggml's op: it replaces the host-side shift plus the attention node. */
int vxfa_flash_attn_ext_ring(vxfa_ctx* ctx, const vxfa_tensor* q,
                             vxfa_tensor* k, vxfa_tensor* v,
                             const vxfa_ring* ring, const vxfa_tensor* k_new,
                             const vxfa_tensor* v_new, vxfa_tensor* dst,
                             float scale, float max_bias, float logit_softcap,
                             void* stream);

/* Rotary embedding fused into the op. build_decoder_layer rotates Q and K
 * with ggml_rope_ext (src/voxtral.cpp:1746-1749: mode 0, n_dims = head dim,
 * freq_base = the decoder's rope theta, freq_scale 1, ext_factor 0,
 * attn_factor 1), copies them contiguous (:1752-1753), stores K and V in
 * the cache (:1758-1770) and attends (:1802); the realtime encoder rotates
 * Q and K the same way with its own theta (:1595-1598). Pair j = dims
 * (2j, 2j+1) of a head at position p turns by theta_j, theta_0 = p and
 * theta_{j+1} = theta_j * freq_base^(-2 / n_dims) (ggml's running product),
 * x0' = x0 cos - x1 sin, x1' = x0 sin + x1 cos; dims >= n_dims are not
 * rotated. */
typedef struct vxfa_rope {
    const int32_t* positions;  /* device; token i of batch b: positions[b * Nq + i] */
    int32_t n_dims;            /* rotated leading dims of each head (even, <= D)      */
    int32_t mode;              /* 0 (ggml's GGML_ROPE_TYPE_NORMAL: adjacent pairs)    */
    float   freq_base;         /* rope theta                                          */
    float   freq_scale;        /* 1                                                   */
} vxfa_rope;

/* The op on unrotated inputs: rotate q (F32 [D, Nq, Hq, B]) and the new K
 * rows, append the new rows (k_new, v_new F32 [Hkv * D, Nq, 1, B]: the new
 * rows are the query tokens, at the last Nq rows of the F16 views k, v),
 * then attend. Equals vxfa_flash_attn_ext_append(rope(q), k, v, rope(k_new),
 * v_new, mask, ...) within the rounding of cos / sin. A decode step is one
 * launch; otherwise the append (with K rotation) runs first. No counterpart
 * in ggml's op: it replaces the two rope nodes, their contiguous copies, the
 * two cache copies and the attention node of a layer. */
int vxfa_flash_attn_ext_rope(vxfa_ctx* ctx, const vxfa_tensor* q,
                             vxfa_tensor* k, vxfa_tensor* v,
                             const vxfa_tensor* k_new,
                             const vxfa_tensor* v_new, const vxfa_rope* rope,
                             const vxfa_tensor* mask, vxfa_tensor* dst,
                             float scale, float max_bias, float logit_softcap,
                             void* stream);

/* GGML_OP_FLASH_ATTN_EXT without a context and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory or create a context at that point (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * contract, results and status codes as vxfa_flash_attn_ext, on the current
 * HIP device and `stream`; the scratch it needs (split-KV partial records of
 * a decode step, f16 staging of F32 K/V for a prefill call) lives in a
 * static 8 MiB array in the library's code object, one per GPU, kept until
 * the process ends. Limits: F32 K/V prefill calls whose f16 K and V exceed
 * 8 MiB return VXFA_NO_WORKSPACE; decode steps always run (with fewer
 * splits if their records would not fit, which the call shapes of voxtral
 * never reach). Every call on one GPU shares the array, so calls that
 * overlap on one GPU race. Its messages are read with vxfa_last_error(NULL)
 * (per calling thread). */
int vxfa_flash_attn_ext_noalloc(const vxfa_tensor* q, const vxfa_tensor* k,
                                const vxfa_tensor* v, const vxfa_tensor* mask,
                                vxfa_tensor* dst, float scale, float max_bias,
                                float logit_softcap, void* stream);

/* Human-readable name of a status code (static storage). */
const char* vxfa_status_str(int status);

/* Message for the last failing call on this context ("" if none); with
 * NULL, for the calling thread's last vxfa_flash_attn_ext_noalloc call. */
const char* vxfa_last_error(const vxfa_ctx* ctx);

/* Library version: major * 10000 + minor * 100 + patch. */
int vxfa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* VXFA_H */
