/*
 * fa_cpu_simd.c — TEST INFRASTRUCTURE ONLY (CPU baseline timed by bench.py).
 *
 * ggml's one-row GGML_OP_FLASH_ATTN_EXT CPU algorithm (restated scalar in
 * fa_oracle.c, which stays the parity checker) with the vector kernels
 * ggml-cpu uses on x86 with AVX2 + FMA + F16C, so that the timed baseline is
 * the shape of the reference's CPU path rather than a scalar restatement:
 *
 *   per (q row iq1, head iq2, batch iq3), rows split over threads:
 *     Q row -> f16 (vcvtps2ph, round to nearest even)
 *     VKQ16 = 0 (f16), M = -inf, S = 0
 *     for each kv position: mask -inf -> skip
 *       s = vec_dot_f16(K row, Qh) * scale + mask     8-wide F16C loads, four
 *                                                     FMA accumulators (32
 *                                                     elements per step)
 *       s > M: M = s, ms = expf(Mold - M), VKQ16 *= ms (vec_scale_f16)
 *       else : vs = expf(s - M)
 *       VKQ16 += vs * V row                           vec_mad_f16: f16 -> f32,
 *                                                     FMA, f32 -> f16 (RNE)
 *       S = S * ms + vs
 *     dst = VKQ16 * (S == 0 ? 0 : 1 / S)
 *
 * ggml lives outside the reference tree (ggml-org/ggml@5cecdad, fetched at
 * configure time by CMakeLists.txt:29-39) and is absent here, so this file
 * follows ggml's published vec.h / simd-mappings.h behaviour for f16 data
 * (GGML_F16_STEP 32, GGML_F16_EPR 8) in code of its own. The reference
 * builds ggml-cpu with -march=native (CMakeLists.txt:83); this file is built
 * for x86-64-v3 (AVX2, FMA, F16C) so the one binary runs on every host the
 * bench meets. Summation order differs from the scalar oracle (results are
 * within float rounding, checked by tests/test_oracle.py).
 *
 * K and V must be F16 here (the configured cache); Q F32 or F16; mask F16.
 */
#include "fa_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static inline float hsum8(__m256 v) {
    const __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

static inline __m256 load_h8(const uint16_t* p) { return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)p)); }
static inline void store_h8(uint16_t* p, __m256 x) {
    _mm_storeu_si128((__m128i*)p, _mm256_cvtps_ph(x, _MM_FROUND_TO_NEAREST_INT));
}

/* ggml_vec_dot_f16: four 8-lane accumulators over 32-element steps, then a
 * pairwise reduction; scalar tail */
static float vec_dot_f16(const uint16_t* x, const uint16_t* y, int64_t n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
    int64_t i = 0;
    for (; i + 32 <= n; i += 32) {
        a0 = _mm256_fmadd_ps(load_h8(x + i), load_h8(y + i), a0);
        a1 = _mm256_fmadd_ps(load_h8(x + i + 8), load_h8(y + i + 8), a1);
        a2 = _mm256_fmadd_ps(load_h8(x + i + 16), load_h8(y + i + 16), a2);
        a3 = _mm256_fmadd_ps(load_h8(x + i + 24), load_h8(y + i + 24), a3);
    }
    float s = hsum8(_mm256_add_ps(_mm256_add_ps(a0, a2), _mm256_add_ps(a1, a3)));
    for (; i < n; ++i) s += oracle_f16_to_f32(x[i]) * oracle_f16_to_f32(y[i]);
    return s;
}

/* ggml_vec_mad_f16: y += x * v, y stored as f16 */
static void vec_mad_f16(int64_t n, uint16_t* y, const uint16_t* x, float v) {
    const __m256 vv = _mm256_set1_ps(v);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) store_h8(y + i, _mm256_fmadd_ps(load_h8(x + i), vv, load_h8(y + i)));
    for (; i < n; ++i) y[i] = oracle_f32_to_f16(fmaf(oracle_f16_to_f32(x[i]), v, oracle_f16_to_f32(y[i])));
}

/* ggml_vec_scale_f16: y *= v, y stored as f16 */
static void vec_scale_f16(int64_t n, uint16_t* y, float v) {
    const __m256 vv = _mm256_set1_ps(v);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) store_h8(y + i, _mm256_mul_ps(load_h8(y + i), vv));
    for (; i < n; ++i) y[i] = oracle_f32_to_f16(oracle_f16_to_f32(y[i]) * v);
}

typedef struct {
    const vxfa_tensor *q, *k, *v, *mask;
    vxfa_tensor* dst;
    float scale;
} simd_job_t;

typedef struct {
    const simd_job_t* job;
    int64_t r0, r1;
} simd_span_t;

static void* simd_rows(void* arg) {
    const simd_span_t* sp = (const simd_span_t*)arg;
    const simd_job_t* J = sp->job;
    const vxfa_tensor *q = J->q, *k = J->k, *v = J->v, *mask = J->mask;
    const int64_t DK = k->ne[0], DV = v->ne[0];
    const int64_t Nq = q->ne[1], Hq = q->ne[2];
    const int64_t nkv = k->ne[1];
    const int64_t rk2 = q->ne[2] / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    uint16_t* Qh = (uint16_t*)aligned_alloc(64, sizeof(uint16_t) * (size_t)((DK + 31) & ~31));
    uint16_t* VKQ16 = (uint16_t*)aligned_alloc(64, sizeof(uint16_t) * (size_t)((DV + 31) & ~31));
    for (int64_t ir = sp->r0; ir < sp->r1; ++ir) {
        const int64_t iq3 = ir / (Hq * Nq);
        const int64_t iq2 = (ir - iq3 * Hq * Nq) / Nq;
        const int64_t iq1 = ir - iq3 * Hq * Nq - iq2 * Nq;
        const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3;
        const char* qrow = (const char*)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3];
        if (q->type == VXFA_TYPE_F16) {
            memcpy(Qh, qrow, sizeof(uint16_t) * (size_t)DK);
        } else {
            const float* qf = (const float*)qrow;
            int64_t d = 0;
            for (; d + 8 <= DK; d += 8) store_h8(Qh + d, _mm256_loadu_ps(qf + d));
            for (; d < DK; ++d) Qh[d] = oracle_f32_to_f16(qf[d]);
        }
        const uint16_t* mp = NULL;
        if (mask)
            mp = (const uint16_t*)((const char*)mask->data + iq1 * mask->nb[1] + (iq2 % mask->ne[2]) * mask->nb[2] +
                                   (iq3 % mask->ne[3]) * mask->nb[3]);
        memset(VKQ16, 0, sizeof(uint16_t) * (size_t)DV);
        float S = 0.0f, M = -INFINITY;
        const char* kbase = (const char*)k->data + ik2 * k->nb[2] + ik3 * k->nb[3];
        const char* vbase = (const char*)v->data + ik2 * v->nb[2] + ik3 * v->nb[3];
        for (int64_t ic = 0; ic < nkv; ++ic) {
            const float mv = mp ? oracle_f16_to_f32(mp[ic]) : 0.0f;
            if (mv == -INFINITY) continue;
            float s = vec_dot_f16((const uint16_t*)(kbase + ic * k->nb[1]), Qh, DK);
            s = s * J->scale + mv;
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                vec_scale_f16(DV, VKQ16, ms);
            } else {
                vs = expf(s - M);
            }
            vec_mad_f16(DV, VKQ16, (const uint16_t*)(vbase + ic * v->nb[1]), vs);
            S = S * ms + vs;
        }
        const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
        float* out = (float*)((char*)J->dst->data + ((iq3 * Nq + iq1) * Hq + iq2) * J->dst->nb[1]);
        int64_t d = 0;
        const __m256 si = _mm256_set1_ps(S_inv);
        for (; d + 8 <= DV; d += 8) _mm256_storeu_ps(out + d, _mm256_mul_ps(load_h8(VKQ16 + d), si));
        for (; d < DV; ++d) out[d] = oracle_f16_to_f32(VKQ16[d]) * S_inv;
    }
    free(Qh);
    free(VKQ16);
    return NULL;
}

/* A persistent pool of worker threads, as ggml's CPU backend keeps one
 * between graph nodes: workers spin on a generation counter (sleeping
 * briefly once idle for long), so a call does not pay thread creation. */
typedef struct {
    pthread_t tid[256];
    int n;                       /* threads including the caller */
    atomic_uint gen;             /* bumped once per call */
    atomic_int done;             /* workers finished with this call */
    atomic_int stop;
    simd_span_t* spans;
} pool_t;

static pool_t g_pool;
static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;

/* each worker starts from the generation current when it was created, so a
 * call issued before the thread first runs is not missed */
typedef struct { int ith; unsigned gen0; } worker_arg_t;
static worker_arg_t g_wargs[256];

static void* pool_worker(void* p) {
    const int ith = ((worker_arg_t*)p)->ith;
    unsigned seen = ((worker_arg_t*)p)->gen0;
    for (;;) {
        long spins = 0;
        unsigned g;
        while ((g = atomic_load_explicit(&g_pool.gen, memory_order_acquire)) == seen) {
            if (atomic_load(&g_pool.stop)) return NULL;
            if (++spins < 200000) {
                _mm_pause();
            } else {
                struct timespec ts = {0, 50000};
                nanosleep(&ts, NULL);
            }
        }
        seen = g;
        if (atomic_load(&g_pool.stop)) return NULL;
        simd_rows(&g_pool.spans[ith]);
        atomic_fetch_add_explicit(&g_pool.done, 1, memory_order_release);
    }
}

static void pool_resize(int n) {
    if (g_pool.n == n) return;
    if (g_pool.n > 1) {
        atomic_store(&g_pool.stop, 1);
        atomic_fetch_add(&g_pool.gen, 1);
        for (int t = 1; t < g_pool.n; ++t) pthread_join(g_pool.tid[t], NULL);
    }
    atomic_store(&g_pool.stop, 0);
    atomic_store(&g_pool.done, 0);
    g_pool.n = n;
    const unsigned gen0 = atomic_load(&g_pool.gen);
    for (int t = 1; t < n; ++t) {
        g_wargs[t].ith = t;
        g_wargs[t].gen0 = gen0;
        pthread_create(&g_pool.tid[t], NULL, pool_worker, &g_wargs[t]);
    }
}

int oracle_fa_cpu_simd(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                       const vxfa_tensor* mask, vxfa_tensor* dst, float scale, int n_threads) {
    if (!q || !k || !v || !dst) return -1;
    if (k->type != VXFA_TYPE_F16 || v->type != VXFA_TYPE_F16 || dst->type != VXFA_TYPE_F32) return -1;
    if (q->type != VXFA_TYPE_F32 && q->type != VXFA_TYPE_F16) return -1;
    if (k->nb[0] != 2 || v->nb[0] != 2 || q->nb[0] != (size_t)(q->type == VXFA_TYPE_F32 ? 4 : 2)) return -1;
    if (q->ne[0] != k->ne[0] || k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3]) return -1;
    if (k->ne[2] <= 0 || k->ne[3] <= 0 || q->ne[2] % k->ne[2] || q->ne[3] % k->ne[3]) return -1;
    if (mask && (mask->type != VXFA_TYPE_F16 || mask->nb[0] != 2 || mask->ne[0] != k->ne[1] ||
                 mask->ne[1] < q->ne[1] || mask->ne[2] <= 0 || mask->ne[3] <= 0 || q->ne[2] % mask->ne[2] ||
                 q->ne[3] % mask->ne[3]))
        return -1;
    if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != q->ne[3] ||
        dst->nb[1] != 4 * (size_t)dst->ne[0])
        return -1;
    const int64_t nrows = q->ne[1] * q->ne[2] * q->ne[3];
    if (nrows == 0) return 0;
    simd_job_t J = {q, k, v, mask, dst, scale};
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    simd_span_t spans[256];
    /* rows split into n_threads contiguous chunks (some may be empty) */
    const int64_t per = (nrows + n_threads - 1) / n_threads;
    for (int t = 0; t < n_threads; ++t) {
        spans[t].job = &J;
        spans[t].r0 = t * per < nrows ? t * per : nrows;
        spans[t].r1 = (t + 1) * per < nrows ? (t + 1) * per : nrows;
    }
    pthread_mutex_lock(&g_pool_mu);
    pool_resize(n_threads);
    g_pool.spans = spans;
    atomic_store(&g_pool.done, 0);
    atomic_fetch_add_explicit(&g_pool.gen, 1, memory_order_release);
    simd_rows(&spans[0]);
    while (atomic_load_explicit(&g_pool.done, memory_order_acquire) < n_threads - 1) _mm_pause();
    pthread_mutex_unlock(&g_pool_mu);
    return 0;
}
