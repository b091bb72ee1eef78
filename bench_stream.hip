// bench_stream.hip — measurement helper for bench.py (not part of the op):
// a read-only HBM stream, the reference rate the decode kernels' GB/s are
// compared with. Each thread keeps eight 16-byte loads in flight per round
// (grid-stride), folds them with XOR and stores only when the fold hits a
// value the data never produces, so the reads cannot be elided and the
// kernel writes (almost) nothing. 512 workgroups of 256 threads: a 32 MiB
// buffer is 16 loads per thread, two rounds of eight.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, int64_t n16, uint32_t* out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (; i + 7 * stride < n16; i += 8 * stride) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= p[i];
    const uint32_t f = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (f == 0x9E3779B9u) out[0] = f;
}

extern "C" int bench_stream_read(const void* buf, int64_t nbytes, void* out, void* stream) {
    const int64_t n16 = nbytes / 16;
    hipLaunchKernelGGL(stream_read_kernel, dim3(512), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(buf), n16, static_cast<uint32_t*>(out));
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
