// fa_kv_append.hip — appends new K and V rows to an f16 KV cache.
//
// Replaces the two ggml_cpy nodes of build_decoder_layer that store the
// layer's new keys and values in the cache (src/voxtral.cpp:1758-1770) when
// the cache is F16: each F32 element is rounded to f16 (round to nearest
// even, overflow to inf, the F16C conversion ggml's CPU copy uses). One
// launch writes K and V: workgroup (t, b) writes token t of kv batch b, each
// thread converts 8 consecutive elements (two 16-byte loads, one 16-byte
// store). The source row is Hkv * D floats, kv head h at h * D (the layout of
// the reshape at :1743); the cache row of head h is the view's (pos, h) row.
// With rope_pos set, K rows are first turned by the rotary embedding of
// their token's position (ggml_rope_ext mode 0, :1748-1749), as the
// reference rotates K before storing it.
#include "fa_common.h"

namespace vxfa {

__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
    const int t = blockIdx.x, b = blockIdx.y;
    const int per = a.hkv * a.d / 8;   // 8-element chunks per matrix row
    // the token's rotary cos / sin per pair, shared by its kv heads
    __shared__ float2 cs[128];
    if (a.rope_pos) {
        const int p = a.rope_pos[b * a.n_new + t];
        // (pairs below 64: one unrolled running product shared by the lanes)
        for (int j = threadIdx.x; j < a.d / 2; j += 256)
            cs[j] = j < 64 ? rope_cs_chain<64>(p, j, a.rope_ts) : rope_cs(p, j, a.rope_ts);
        __syncthreads();
    }
    for (int c = threadIdx.x; c < 2 * per; c += 256) {
        const bool is_v = c >= per;
        const int e = 8 * (is_v ? c - per : c);
        const int h = e / a.d, d = e - h * a.d;
        const float* src = is_v ? a.v_new : a.k_new;
        const int64_t soff = (int64_t)t * (is_v ? a.vn_nb1 : a.kn_nb1) + (int64_t)b * (is_v ? a.vn_nb3 : a.kn_nb3);
        const floatx4* sp = (const floatx4*)((const char*)src + soff) + e / 4;
        const floatx4 x0 = sp[0], x1 = sp[1];
        float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        if (!is_v && a.rope_pos) rope8_tab(x, d, cs, a.rope_dims);
        half8 y;
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = (_Float16)x[i];
        const int64_t pos = (int64_t)a.pos0 + t;
        char* dst = is_v ? (char*)a.v + pos * a.v_nb1 + (int64_t)h * a.v_nb2 + (int64_t)b * a.v_nb3
                         : (char*)a.k + pos * a.k_nb1 + (int64_t)h * a.k_nb2 + (int64_t)b * a.k_nb3;
        *(half8*)(dst + 2 * d) = y;
    }
}

hipError_t launch_kv_append(const AppendArgs& a, hipStream_t st) {
    if (a.n_new <= 0 || a.bk <= 0) return hipSuccess;
    if (a.d % 8 || a.d > 256 || a.bk > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)a.n_new, (unsigned)a.bk), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace vxfa
