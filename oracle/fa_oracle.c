/*
 * fa_oracle.c — TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline).
 *
 * CPU restatement of ggml's GGML_OP_FLASH_ATTN_EXT as voxtral.cpp uses it.
 * The arithmetic of that op lives in ggml, an external dependency pinned at
 * ggml-org/ggml@5cecdad692d868e28dbd2f7c468504770108f30c (reference
 * CMakeLists.txt:29-39); ggml is not part of the reference tree and cannot be
 * fetched here, so the published one-row CPU algorithm of
 * ggml/src/ggml-cpu/ops.cpp (ggml_compute_forward_flash_attn_ext_f16_one_chunk)
 * is restated from its documented behaviour:
 *
 *   for each (q row iq1, head iq2, batch iq3):          rows split over threads
 *     Qq   = Q row converted to K's dot type (f16 when K is f16)
 *     M = -inf, S = 0, VKQ = 0 (f16 array when V is f16, else f32)
 *     for each kv position ic:
 *       mv = mask[ic]                  (0 when no mask)
 *       if mv == -inf: skip the position
 *       s  = dot(K row, Qq) * scale
 *       s += mv
 *       if s > M: M = s, ms = exp(Mold - M), VKQ *= ms, vs = 1
 *       else    : ms = 1, vs = exp(s - M)
 *       VKQ += vs * V row;  S = S * ms + vs
 *     dst[iq3][iq1][iq2] = VKQ * (S == 0 ? 0 : 1/S)    (permuted layout)
 *
 * Call sites whose tensor views this follows: src/voxtral.cpp:1580-1613
 * (encoder, mask = NULL, scale = 1/sqrt(hd)) and :1736-1805 (decoder GQA
 * views over the token-major KV cache, mask cast to F16 at :1801). Mask
 * values come from :2104-2111 (causal) and :2179-2190 (encoder window).
 * Thread count default in the reference: min(hw, 16) at :1046-1051.
 *
 * voxtral passes max_bias = 0 and logit_softcap = 0 at both call sites, and
 * the HIP path reports anything else as unsupported; ggml's ALiBi slope and
 * tanh soft-capping are therefore not restated here, and both routines
 * reject nonzero values as a contract violation.
 *
 * The f64 routine is an exact two-pass softmax used to pin the restatement.
 */
#include "fa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* binary16 conversions (IEEE 754-2008, round to nearest, ties to even) */

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in binary32 */
        const float mag = (float)m * 0x1p-24f;
        return float_of(bits_of(mag) | sign);
    }
    if (e == 31) return float_of(sign | 0x7f800000u | (m << 13));
    return float_of(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    const uint32_t x = bits_of(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN stays NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {
        /* result is subnormal (or rounds up to the smallest normal):
         * mantissa = round_even(|f| / 2^-24); the scaling is exact */
        const float scaled = float_of(ax) * 0x1p24f;
        const uint32_t mi = (uint32_t)nearbyintf(scaled);
        return (uint16_t)(sign | mi);
    }
    uint32_t r = ((ax >> 23) - 112u) << 10 | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1u; /* carry may bump the exponent: correct */
    return (uint16_t)(sign | r);
}

void oracle_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}

void oracle_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------ */
/* contract checks shared by both routines */

static int elt_size(int32_t t) { return t == VXFA_TYPE_F32 ? 4 : (t == VXFA_TYPE_F16 ? 2 : 0); }

static int check_contract(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                          const vxfa_tensor* mask, const vxfa_tensor* dst, int dst_f32) {
    if (!q || !k || !v) return -1;
    if (!elt_size(q->type) || !elt_size(k->type) || !elt_size(v->type)) return -1;
    if (q->nb[0] != (size_t)elt_size(q->type) || k->nb[0] != (size_t)elt_size(k->type) ||
        v->nb[0] != (size_t)elt_size(v->type)) return -1;
    if (q->ne[0] != k->ne[0]) return -1;
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3]) return -1;
    if (k->ne[2] <= 0 || k->ne[3] <= 0) return -1;
    if (q->ne[2] % k->ne[2] || q->ne[3] % k->ne[3]) return -1;
    if (mask) {
        if (mask->type != VXFA_TYPE_F16 || mask->nb[0] != 2) return -1;
        if (mask->ne[0] != k->ne[1] || mask->ne[1] < q->ne[1]) return -1;
        if (mask->ne[2] <= 0 || mask->ne[3] <= 0) return -1;
        if (q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3]) return -1;
    }
    if (dst) {
        if (dst_f32 && dst->type != VXFA_TYPE_F32) return -1;
        if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] ||
            dst->ne[3] != q->ne[3]) return -1;
        if (dst->nb[0] != 4 || dst->nb[1] != dst->nb[0] * (size_t)dst->ne[0] ||
            dst->nb[2] != dst->nb[1] * (size_t)dst->ne[1] ||
            dst->nb[3] != dst->nb[2] * (size_t)dst->ne[2]) return -1;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* threading helper */

typedef struct {
    void (*fn)(void* arg, int64_t r0, int64_t r1, int ith);
    void* arg;
    int64_t r0, r1;
    int ith;
} span_t;

static void* span_main(void* p) {
    span_t* s = (span_t*)p;
    s->fn(s->arg, s->r0, s->r1, s->ith);
    return NULL;
}

static void parallel_rows(int64_t nrows, int n_threads,
                          void (*fn)(void*, int64_t, int64_t, int), void* arg) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    if ((int64_t)n_threads > nrows) n_threads = (int)(nrows > 0 ? nrows : 1);
    span_t spans[256];
    pthread_t tids[256];
    const int64_t per = (nrows + n_threads - 1) / n_threads;
    for (int t = 0; t < n_threads; ++t) {
        spans[t].fn = fn; spans[t].arg = arg; spans[t].ith = t;
        spans[t].r0 = t * per < nrows ? t * per : nrows;
        spans[t].r1 = (t + 1) * per < nrows ? (t + 1) * per : nrows;
    }
    for (int t = 1; t < n_threads; ++t) pthread_create(&tids[t], NULL, span_main, &spans[t]);
    span_main(&spans[0]);
    for (int t = 1; t < n_threads; ++t) pthread_join(tids[t], NULL);
}

/* ------------------------------------------------------------------ */
/* ggml-faithful one-row algorithm */

typedef struct {
    const vxfa_tensor *q, *k, *v, *mask;
    vxfa_tensor* dst;
    float scale;
    int flags;
} ggml_job_t;

/* dot product with 32 running partial sums combined pairwise, the shape of
 * ggml's SIMD dot (four 8-lane accumulators); the order is not bit-pinned */
static float dot_f16(const uint16_t* a, const uint16_t* b, int64_t n) {
    float acc[32] = {0};
    int64_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 32; ++j)
            acc[j] = fmaf(oracle_f16_to_f32(a[i + j]), oracle_f16_to_f32(b[i + j]), acc[j]);
    for (int w = 16; w >= 1; w >>= 1)
        for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
    float s = acc[0];
    for (; i < n; ++i) s += oracle_f16_to_f32(a[i]) * oracle_f16_to_f32(b[i]);
    return s;
}

static float dot_f32(const float* a, const float* b, int64_t n) {
    float acc[32] = {0};
    int64_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 32; ++j) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    for (int w = 16; w >= 1; w >>= 1)
        for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
    float s = acc[0];
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

static float load_elt(const char* p, int32_t type) {
    if (type == VXFA_TYPE_F32) { float f; memcpy(&f, p, 4); return f; }
    uint16_t h; memcpy(&h, p, 2); return oracle_f16_to_f32(h);
}

static void ggml_rows(void* arg, int64_t ir0, int64_t ir1, int ith) {
    (void)ith;
    const ggml_job_t* J = (const ggml_job_t*)arg;
    const vxfa_tensor *q = J->q, *k = J->k, *v = J->v, *mask = J->mask;
    const int64_t DK = k->ne[0], DV = v->ne[0];
    const int64_t Nq = q->ne[1], Hq = q->ne[2];
    const int64_t nkv = k->ne[1];
    const int64_t rk2 = q->ne[2] / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    const int flags = J->flags;

    float scale = J->scale;
    if (flags & ORACLE_MUT_NO_SCALE) scale = 1.0f;

    const int k_f16 = k->type == VXFA_TYPE_F16;
    const int v_f16 = v->type == VXFA_TYPE_F16;
    const int vkq16 = v_f16 && (flags & ORACLE_VKQ_F16);

    float* Qf = (float*)malloc(sizeof(float) * DK);
    uint16_t* Qh = (uint16_t*)malloc(sizeof(uint16_t) * DK);
    float* VKQ32 = (float*)malloc(sizeof(float) * DV);
    uint16_t* VKQ16 = (uint16_t*)malloc(sizeof(uint16_t) * DV);
    float* Kf = (float*)malloc(sizeof(float) * DK);

    for (int64_t ir = ir0; ir < ir1; ++ir) {
        const int64_t iq3 = ir / (Hq * Nq);
        const int64_t iq2 = (ir - iq3 * Hq * Nq) / Nq;
        const int64_t iq1 = ir - iq3 * Hq * Nq - iq2 * Nq;

        const int64_t ik2 = (flags & ORACLE_MUT_GQA_MOD) ? iq2 % k->ne[2] : iq2 / rk2;
        const int64_t ik3 = iq3 / rk3;

        const char* qrow = (const char*)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3];
        for (int64_t d = 0; d < DK; ++d) Qf[d] = load_elt(qrow + d * q->nb[0], q->type);
        if (k_f16) for (int64_t d = 0; d < DK; ++d) Qh[d] = oracle_f32_to_f16(Qf[d]);

        const uint16_t* mp = NULL;
        if (mask && !(flags & ORACLE_MUT_NO_MASK))
            mp = (const uint16_t*)((const char*)mask->data + iq1 * mask->nb[1] +
                                   (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3]);

        float S = 0.0f, M = -INFINITY;
        if (vkq16) memset(VKQ16, 0, sizeof(uint16_t) * DV);
        else memset(VKQ32, 0, sizeof(float) * DV);

        for (int64_t ic = 0; ic < nkv; ++ic) {
            const float mv = mp ? oracle_f16_to_f32(mp[ic]) : 0.0f;
            if (mv == -INFINITY) continue;

            const char* krow = (const char*)k->data + ic * k->nb[1] + ik2 * k->nb[2] + ik3 * k->nb[3];
            float s;
            if (k_f16) {
                s = dot_f16((const uint16_t*)krow, Qh, DK);
            } else {
                memcpy(Kf, krow, sizeof(float) * DK);
                s = dot_f32(Kf, Qf, DK);
            }
            s = s * scale;
            s += mv;

            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            int64_t icv = ic;
            if ((flags & ORACLE_MUT_V_SHIFT) && ic + 1 < nkv) icv = ic + 1;
            const char* vrow = (const char*)v->data + icv * v->nb[1] + ik2 * v->nb[2] + ik3 * v->nb[3];

            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                if (flags & ORACLE_MUT_NO_MAXSUB) ms = 1.0f;
                if (vkq16) {
                    for (int64_t d = 0; d < DV; ++d)
                        VKQ16[d] = oracle_f32_to_f16(oracle_f16_to_f32(VKQ16[d]) * ms);
                } else {
                    for (int64_t d = 0; d < DV; ++d) VKQ32[d] *= ms;
                }
            } else {
                vs = expf(s - M);
            }

            if (vkq16) {
                const uint16_t* vh = (const uint16_t*)vrow;
                for (int64_t d = 0; d < DV; ++d)
                    VKQ16[d] = oracle_f32_to_f16(fmaf(oracle_f16_to_f32(vh[d]), vs, oracle_f16_to_f32(VKQ16[d])));
            } else {
                for (int64_t d = 0; d < DV; ++d)
                    VKQ32[d] = fmaf(load_elt(vrow + d * v->nb[0], v->type), vs, VKQ32[d]);
            }
            S = S * ms + vs;
        }

        if (vkq16)
            for (int64_t d = 0; d < DV; ++d) VKQ32[d] = oracle_f16_to_f32(VKQ16[d]);

        const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
        float* out = (float*)((char*)J->dst->data + ((iq3 * Nq + iq1) * Hq + iq2) * J->dst->nb[1]);
        for (int64_t d = 0; d < DV; ++d) out[d] = VKQ32[d] * S_inv;
    }
    free(Qf); free(Qh); free(VKQ32); free(VKQ16); free(Kf);
}

int oracle_fa_ggml(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                   const vxfa_tensor* mask, vxfa_tensor* dst, float scale, float max_bias,
                   float logit_softcap, int flags, int n_threads) {
    if (check_contract(q, k, v, mask, dst, 1)) return -1;
    if (max_bias != 0.0f || logit_softcap != 0.0f) return -1;
    ggml_job_t J = {q, k, v, mask, dst, scale, flags};
    const int64_t nrows = q->ne[1] * q->ne[2] * q->ne[3];
    if (nrows == 0) return 0;
    parallel_rows(nrows, n_threads, ggml_rows, &J);
    return 0;
}

/* ------------------------------------------------------------------ */
/* exact double-precision reference */

typedef struct {
    const vxfa_tensor *q, *k, *v, *mask;
    double* dst;
    float scale;
    int q_f16;
} f64_job_t;

static void f64_rows(void* arg, int64_t ir0, int64_t ir1, int ith) {
    (void)ith;
    const f64_job_t* J = (const f64_job_t*)arg;
    const vxfa_tensor *q = J->q, *k = J->k, *v = J->v, *mask = J->mask;
    const int64_t DK = k->ne[0], DV = v->ne[0];
    const int64_t Nq = q->ne[1], Hq = q->ne[2];
    const int64_t nkv = k->ne[1];
    const int64_t rk2 = q->ne[2] / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    double* qd = (double*)malloc(sizeof(double) * DK);
    double* sc = (double*)malloc(sizeof(double) * (nkv > 0 ? nkv : 1));
    double* acc = (double*)malloc(sizeof(double) * DV);
    const double scale = (double)J->scale;

    for (int64_t ir = ir0; ir < ir1; ++ir) {
        const int64_t iq3 = ir / (Hq * Nq);
        const int64_t iq2 = (ir - iq3 * Hq * Nq) / Nq;
        const int64_t iq1 = ir - iq3 * Hq * Nq - iq2 * Nq;
        const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3;

        const char* qrow = (const char*)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3];
        for (int64_t d = 0; d < DK; ++d) {
            float f = load_elt(qrow + d * q->nb[0], q->type);
            if (J->q_f16) f = oracle_f16_to_f32(oracle_f32_to_f16(f));
            qd[d] = f;
        }
        const uint16_t* mp = NULL;
        if (mask)
            mp = (const uint16_t*)((const char*)mask->data + iq1 * mask->nb[1] +
                                   (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3]);
        double M = -INFINITY;
        for (int64_t ic = 0; ic < nkv; ++ic) {
            const double mv = mp ? (double)oracle_f16_to_f32(mp[ic]) : 0.0;
            if (mv == -INFINITY) { sc[ic] = -INFINITY; continue; }
            const char* krow = (const char*)k->data + ic * k->nb[1] + ik2 * k->nb[2] + ik3 * k->nb[3];
            double s = 0.0;
            for (int64_t d = 0; d < DK; ++d) s += qd[d] * (double)load_elt(krow + d * k->nb[0], k->type);
            s *= scale;
            s += mv;
            sc[ic] = s;
            if (s > M) M = s;
        }
        for (int64_t d = 0; d < DV; ++d) acc[d] = 0.0;
        double S = 0.0;
        if (M != -INFINITY) {
            for (int64_t ic = 0; ic < nkv; ++ic) {
                if (sc[ic] == -INFINITY) continue;
                const double w = exp(sc[ic] - M);
                S += w;
                const char* vrow = (const char*)v->data + ic * v->nb[1] + ik2 * v->nb[2] + ik3 * v->nb[3];
                for (int64_t d = 0; d < DV; ++d) acc[d] += w * (double)load_elt(vrow + d * v->nb[0], v->type);
            }
        }
        double* out = J->dst + ((iq3 * Nq + iq1) * Hq + iq2) * DV;
        for (int64_t d = 0; d < DV; ++d) out[d] = S == 0.0 ? 0.0 : acc[d] / S;
    }
    free(qd); free(sc); free(acc);
}

int oracle_fa_f64(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                  const vxfa_tensor* mask, double* dst, float scale, float max_bias,
                  float logit_softcap, int q_f16, int n_threads) {
    if (!dst || check_contract(q, k, v, mask, NULL, 0)) return -1;
    if (max_bias != 0.0f || logit_softcap != 0.0f) return -1;
    f64_job_t J = {q, k, v, mask, dst, scale, q_f16};
    const int64_t nrows = q->ne[1] * q->ne[2] * q->ne[3];
    if (nrows == 0) return 0;
    parallel_rows(nrows, n_threads, f64_rows, &J);
    return 0;
}
