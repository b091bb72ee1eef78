// fa_common.h — shared device helpers and launch descriptors for the gfx950
// attention kernels. CDNA4 only: 64-lane wavefronts, MFMA f16 tiles, LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vxfa {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr uint16_t kF16NegInf = 0xFC00u;

// Everything a kernel needs from the ggml descriptors, in elements where the
// row is contiguous and in bytes for the outer strides.
struct AttnArgs {
    const void* q;        // F32 or F16
    const _Float16* k;
    const _Float16* v;
    const uint16_t* mask; // F16 bits, may be null
    float* dst;           // [B][Nq][Hq][D]
    float* ws;            // split-KV partials (decode)
    int64_t q_nb1, q_nb2, q_nb3;   // bytes
    int64_t k_nb1, k_nb2, k_nb3;   // bytes
    int64_t v_nb1, v_nb2, v_nb3;   // bytes
    int64_t m_nb1, m_nb2, m_nb3;   // bytes
    int32_t nq, nkv, hq, hkv, b, bk, hm, bm;
    int32_t q_f16;        // q element type is f16
    int32_t n_split;      // decode: workgroups per (batch, kv head)
    int32_t mask_vec;     // mask data and strides 16-byte aligned (128-bit mask loads)
    float scale_log2;     // scale * log2(e)
};

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// Load 8 consecutive Q elements (F32 or F16) and round them to f16 (RNE),
// the conversion ggml applies to Q before an f16 K dot product.
__device__ __forceinline__ half8 load_q8(const void* base, int64_t byte_off, bool q_f16) {
    half8 r;
    if (q_f16) {
        r = *(const half8*)((const char*)base + byte_off);
    } else {
        const floatx4* p = (const floatx4*)((const char*)base + byte_off);
        floatx4 a = p[0], c = p[1];
        r[0] = (_Float16)a[0]; r[1] = (_Float16)a[1]; r[2] = (_Float16)a[2]; r[3] = (_Float16)a[3];
        r[4] = (_Float16)c[0]; r[5] = (_Float16)c[1]; r[6] = (_Float16)c[2]; r[7] = (_Float16)c[3];
    }
    return r;
}

// Cross-lane helpers over a 64-lane wavefront.
__device__ __forceinline__ float shfl_xor(float x, int m) { return __shfl_xor(x, m, 64); }

// DPP row rotate: lane i of each 16-lane row reads lane (i + n) mod 16 of the
// same row (dpp_ctrl ROW_ROR = 0x120 + n). A VALU operand modifier, no LDS.
template <int N>
__device__ __forceinline__ float row_ror(float x) {
    static_assert(N >= 1 && N <= 15, "rotate amount");
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + N, 0xF, 0xF,
                                                                 false));
}

// max / sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15); every lane
// of the row receives the result
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, row_ror<8>(x));
    x = fmaxf(x, row_ror<4>(x));
    x = fmaxf(x, row_ror<2>(x));
    x = fmaxf(x, row_ror<1>(x));
    return x;
}
__device__ __forceinline__ float row16_sum(float x) {
    x += row_ror<8>(x);
    x += row_ror<4>(x);
    x += row_ror<2>(x);
    x += row_ror<1>(x);
    return x;
}

// Eight consecutive F16 mask entries starting at p, as four 32-bit words
// (entry e in half e % 2 of word e / 2). Entries at or past `valid` read as
// -inf. The widest load the address allows is used: 16, 4 or 2 bytes.
__device__ __forceinline__ u32x4 load_mask8(const uint16_t* p, int valid) {
    const uint32_t dead = 0xFC00FC00u;
    u32x4 w = {dead, dead, dead, dead};
    const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
    if (valid >= 8 && (addr & 15) == 0) {
        w = *reinterpret_cast<const u32x4*>(p);
    } else if (valid >= 8 && (addr & 3) == 0) {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
        w = u32x4{q[0], q[1], q[2], q[3]};
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t h = e < valid ? (uint32_t)p[e] : (uint32_t)kF16NegInf;
            w[e >> 1] = (e & 1) ? ((w[e >> 1] & 0xFFFFu) | (h << 16)) : ((w[e >> 1] & 0xFFFF0000u) | h);
        }
    }
    return w;
}

// Bit e set when entry e of the eight is not -inf.
__device__ __forceinline__ uint32_t live_bits8(u32x4 w) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m |= ((w[i] & 0xFFFFu) != kF16NegInf ? 1u : 0u) << (2 * i);
        m |= ((w[i] >> 16) != kF16NegInf ? 1u : 0u) << (2 * i + 1);
    }
    return m;
}

// Live range [lo, hi) over `rows` mask rows of n entries each (row r at
// base + r * row_stride bytes): lo is the first and hi - 1 the last column
// holding an entry other than -inf in any of the rows; lo = hi = 0 when every
// entry is -inf. Every thread of the block calls it and gets the result.
// Rows are cut into 8-entry chunks; each thread takes whole chunks, four at a
// time with all loads issued before any test, so the scan costs a few memory
// round trips whatever the row alignment. red: 2 ints of LDS per wavefront.
template <int NT>
__device__ __forceinline__ void mask_live_range(const uint16_t* base, int64_t row_stride, int rows, int n, int* red,
                                                int& lo, int& hi) {
    const int tid = threadIdx.x;
    const int nch = (n + 7) >> 3;
    const int items = rows * nch;
    int tlo = 0x7fffffff, thi = -1;
    for (int i0 = tid; i0 < items; i0 += 4 * NT) {
        u32x4 w[4];
        int col[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * NT;
            col[u] = -1;
            w[u] = u32x4{0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u};
            if (i < items) {
                const int r = i / nch, c = i - r * nch;
                col[u] = 8 * c;
                const uint16_t* p = reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(base) +
                                                                      (int64_t)r * row_stride) + 8 * c;
                w[u] = load_mask8(p, n - 8 * c);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t m = live_bits8(w[u]);
            if (m) {
                tlo = min(tlo, col[u] + (int)__builtin_ctz(m));
                thi = max(thi, col[u] + 31 - (int)__builtin_clz(m));
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        tlo = min(tlo, __shfl_xor(tlo, off, 64));
        thi = max(thi, __shfl_xor(thi, off, 64));
    }
    const int wave = tid >> 6;
    if ((tid & 63) == 0) { red[2 * wave] = tlo; red[2 * wave + 1] = thi; }
    __syncthreads();
    tlo = red[0];
    thi = red[1];
#pragma unroll
    for (int wv = 1; wv < NT / 64; ++wv) { tlo = min(tlo, red[2 * wv]); thi = max(thi, red[2 * wv + 1]); }
    __syncthreads();   // red may be reused by the caller
    if (thi < 0) { lo = 0; hi = 0; } else { lo = tlo; hi = thi + 1; }
}

// ---- MFMA tile helpers shared by the prefill kernels ---------------------

typedef short short4v __attribute__((ext_vector_type(4)));

// KV position held by accumulator element j of lane half hh in a 32x32 S^T
// block whose A-operand rows are the K rows permuted so that each half of a
// lane's accumulator covers 8 contiguous positions, in increasing order:
//   hh = 0 : kv = j            hh = 1 : kv = 16 + 4((j / 4 + 2) & 3) + j % 4
__device__ __forceinline__ int pf_kv_of(int hh, int j) {
    return hh ? 16 + (((j >> 2) + 2) & 3) * 4 + (j & 3) : j;
}

// chunk swizzles of the K and V tiles in LDS (r = row within the tile; only
// bits 0-4 matter, so tiles of 32 or more rows share them)
template <int D>
__device__ __forceinline__ int swz_k(int r) {
    return D == 64 ? ((r ^ (r >> 2)) & 7) : (((r >> 1) ^ (r << 2)) & 15);
}
template <int D>
__device__ __forceinline__ int swz_v(int r) {
    return D == 64 ? ((r & 2) << 1) : ((r & 3) << 2);
}

// Four 16-bit elements, transposed across each 16-lane group: lane i of the
// group receives element (i % 4) of the 8 bytes addressed by lane 4r + i/4,
// for r = 0..3 (gfx950 ds_read_b64_tr_b16).
__device__ __forceinline__ half4 lds_read_tr16(const char* p) {
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(p));
    return __builtin_bit_cast(half4, r);
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land
// at LDS offset lds + 16 * l (lds wave-uniform, in M0). Global address:
// uniform base + 32-bit lane offset, or a full 64-bit lane address.
__device__ __forceinline__ void dma16(const char* base, uint32_t off, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma16_addr(const char* addr, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(addr), "{m0}"(lds) : "memory");
}

// wait for every outstanding memory operation of this wavefront
// (s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0))
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

// max / sum over the lane pair (l, l ^ 32): v_permlane32_swap(x, x) returns
// {x[l % 32], x[l % 32 + 32]} in every lane
__device__ __forceinline__ float pair32_max(float x) {
    const int xi = __builtin_bit_cast(int, x);
    const auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
    return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}
__device__ __forceinline__ float pair32_sum(float x) {
    const int xi = __builtin_bit_cast(int, x);
    const auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
    return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}

}  // namespace vxfa

// Host-side launchers (implemented in the kernel translation units).
namespace vxfa {
hipError_t launch_decode(const AttnArgs& a, int head_dim, int group, hipStream_t stream);
constexpr int kDecodeMaxSplit = 64;
constexpr int kDecodeWaves = 4;      // wavefronts per decode split workgroup
// Floats per decode partial record: O [G][D], then m [G] and l [G], padded to
// a multiple of 4 so every record starts 16-byte aligned.
constexpr int dec_record_floats(int D, int G) { return G * D + ((2 * G + 3) & ~3); }
hipError_t launch_prefill(const AttnArgs& a, int head_dim, int waves, hipStream_t stream);
hipError_t launch_prefill64_pp(const AttnArgs& a, int shape, hipStream_t stream);
hipError_t launch_zero(float* dst, int64_t n, hipStream_t stream);
}  // namespace vxfa
