/* ThreadSanitizer run of the oracle's threaded routines: the scalar
 * restatement (threads created per call) and the vectorised baseline (a
 * persistent spinning pool), on a decode-shaped and a prefill-shaped case
 * with several thread counts, twice each so the pool is reused and resized.
 * Built and run by tests/test_sanitizers.py (host code only). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/fa_oracle.h"

static vxfa_tensor view(void* data, int type, int64_t n0, int64_t n1, int64_t n2, int64_t n3, size_t b1, size_t b2,
                        size_t b3) {
    vxfa_tensor t;
    memset(&t, 0, sizeof(t));
    t.data = data;
    t.type = type;
    t.ne[0] = n0; t.ne[1] = n1; t.ne[2] = n2; t.ne[3] = n3;
    t.nb[0] = type == VXFA_TYPE_F32 ? 4 : 2;
    t.nb[1] = b1; t.nb[2] = b2; t.nb[3] = b3;
    return t;
}

int main(void) {
    const int D = 64, H = 4, HK = 2, N = 37, NKV = 53;
    float* q = malloc(sizeof(float) * N * H * D);
    uint16_t* k = malloc(2 * NKV * HK * D);
    uint16_t* v = malloc(2 * NKV * HK * D);
    uint16_t* m = malloc(2 * N * NKV);
    float* o1 = malloc(sizeof(float) * N * H * D);
    float* o2 = malloc(sizeof(float) * N * H * D);
    unsigned s = 7;
    for (int i = 0; i < N * H * D; ++i) { s = s * 1664525u + 1013904223u; q[i] = (float)(s >> 8) / 16777216.f - 0.5f; }
    for (int i = 0; i < NKV * HK * D; ++i) {
        s = s * 1664525u + 1013904223u;
        k[i] = oracle_f32_to_f16((float)(s >> 8) / 16777216.f - 0.5f);
        v[i] = oracle_f32_to_f16((float)(s >> 9) / 8388608.f - 0.5f);
    }
    for (int r = 0; r < N; ++r)
        for (int c = 0; c < NKV; ++c) m[r * NKV + c] = c <= r + 16 ? 0 : 0xFC00u;
    vxfa_tensor tq = view(q, VXFA_TYPE_F32, D, N, H, 1, (size_t)H * D * 4, (size_t)D * 4, (size_t)N * H * D * 4);
    vxfa_tensor tk = view(k, VXFA_TYPE_F16, D, NKV, HK, 1, (size_t)HK * D * 2, (size_t)D * 2, (size_t)NKV * HK * D * 2);
    vxfa_tensor tv = view(v, VXFA_TYPE_F16, D, NKV, HK, 1, (size_t)HK * D * 2, (size_t)D * 2, (size_t)NKV * HK * D * 2);
    vxfa_tensor tm = view(m, VXFA_TYPE_F16, NKV, N, 1, 1, (size_t)NKV * 2, (size_t)N * NKV * 2, (size_t)N * NKV * 2);
    vxfa_tensor t1 = view(o1, VXFA_TYPE_F32, D, H, N, 1, (size_t)D * 4, (size_t)H * D * 4, (size_t)N * H * D * 4);
    vxfa_tensor t2 = view(o2, VXFA_TYPE_F32, D, H, N, 1, (size_t)D * 4, (size_t)H * D * 4, (size_t)N * H * D * 4);
    const int threads[] = {1, 3, 8, 3, 5};
    for (int rep = 0; rep < 5; ++rep) {
        const vxfa_tensor* mk = rep & 1 ? &tm : NULL;
        if (oracle_fa_ggml(&tq, &tk, &tv, mk, &t1, 0.125f, 0.f, 0.f, ORACLE_VKQ_F16, threads[rep])) return 1;
        if (oracle_fa_cpu_simd(&tq, &tk, &tv, mk, &t2, 0.125f, threads[rep])) return 1;
        if (memcmp(o1, o2, sizeof(float) * N * H * D)) { printf("simd != scalar at rep %d\n", rep); return 1; }
    }
    printf("ok\n");
    free(q); free(k); free(v); free(m); free(o1); free(o2);
    return 0;
}
