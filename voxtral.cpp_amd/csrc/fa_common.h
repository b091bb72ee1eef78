// fa_common.h — shared device helpers and launch descriptors for the gfx950
// attention kernels. CDNA4 only: 64-lane wavefronts, MFMA f16 tiles, LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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
    float* ws;            // split-KV partial records (decode)
    int64_t q_nb1, q_nb2, q_nb3;   // bytes
    int64_t k_nb1, k_nb2, k_nb3;   // bytes
    int64_t v_nb1, v_nb2, v_nb3;   // bytes
    int64_t m_nb1, m_nb2, m_nb3;   // bytes
    int32_t nq, nkv, hq, hkv, b, bk, hm, bm;
    int32_t q_f16;        // q element type is f16
    int32_t kv_f32;       // k and v element type is F32 (else f16)
    int32_t n_split;      // decode: workgroups per (batch, kv head)
    int32_t dec_t16;      // decode, f16 K/V: 16-position tiles (short spans) instead of 32
    int32_t mask_vec;     // mask data and strides 16-byte aligned (128-bit mask loads)
    float scale_log2;     // scale * log2(e)
    // implicit causal / window mask (instead of a mask tensor): query row i
    // attends kv j iff j <= i + im_offset and, when im_window > 0,
    // j >= i + im_offset - im_window + 1
    int32_t im_causal;
    int32_t im_window;
    int64_t im_offset;
    // decode without a mask tensor: the live kv range [kv_lo, kv_hi)
    int32_t kv_lo, kv_hi;
    // decode with a fused KV append: the row at n_kv - 1 of k and v is the new
    // token's, taken from the F32 sources k_new / v_new (kv head h at floats
    // h * D .. h * D + D - 1 of the token row; per kv batch nb3 bytes apart),
    // rounded to f16 and also written into k and v
    int32_t append;
    // decode over a ring buffer: logical position p is cache row
    // (ring_start + p) mod ring_cap; 0, 0 = a plain cache
    int32_t ring_start, ring_cap;
    // rotary embedding of Q (and of the appended K rows), ggml's mode 0:
    // position of query row i of batch b at rope_pos[b * nq + i]; rope_pos
    // null = no rotation
    const int32_t* rope_pos;
    float rope_ts;        // theta scale = freq_base^(-2 / n_dims)
    int32_t rope_dims;    // rotated leading dims of each head
    const float* k_new;
    const float* v_new;
    int64_t kn_nb3, vn_nb3;
    // prefill with a mask tensor (the hd 64 pipelined kernel; the short masked
    // prefill after F32 staging): per mask row (batch bm_i, plane p, row q at
    // (bm_i * hm + p) * nq + q) the live interval {lo, hi} when the row is 0
    // on [lo, hi] and -inf elsewhere ({n_kv, -1}: no live entry), else
    // {-2, -2}; written by a pre-pass launch into workspace scratch
    int2* mask_rows;
};

// n / d for 0 <= n < 2^31 by a multiply-high, an add and a shift, with the
// constants computed on the host (Granlund and Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994: s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1, n / d = (mulhi(n, m) + n) >> s, where
// the sum stays below 2^32 because mulhi(n, m) < n < 2^31).
struct FastDiv {
    uint32_t m, s;
    static FastDiv make(uint32_t d) {   // d >= 1
        uint32_t s = 0;
        while ((1ull << s) < d) ++s;
        const uint64_t m = (((1ull << s) - d) << 32) / d + 1;
        return FastDiv{(uint32_t)m, s};
    }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
        return (uint32_t)((((uint64_t)n * m) >> 32) + n) >> s;
    }
};

// Workgroup -> (query tile, head, batch, kv head, kv batch) of a prefill
// grid of nwg = nqt * hq * b workgroups. Workgroups are dealt to the 8 XCDs
// round robin (blockIdx % 8), so logical index gidx is laid out to give each
// XCD a contiguous range: consecutive query tiles of one head then share that
// XCD's L2 for the head's K and V. All constants come from the host, so the
// kernel's first global loads wait on one batch of argument loads and no
// division.
// n / d and n % d for 0 <= n < 2^31, d fixed per launch and set up on the host
// (a division by a run-time value is a long scalar sequence on the GPU, run
// by every wavefront before its first load)
struct DivMod {
    uint32_t d;
    FastDiv f;
    static DivMod make(uint32_t d) { return DivMod{d, FastDiv::make(d)}; }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const { return f.div(n); }
    __host__ __device__ __forceinline__ uint32_t mod(uint32_t n) const { return n - d * f.div(n); }
};

// F32 -> f16 copies of the K and V views [d, n, h, b] (byte strides nb1..nb3,
// rows contiguous) into contiguous [b][n][h][d] f16 buffers dk, dv
struct StageReq {
    const float* k;
    int64_t k_nb1, k_nb2, k_nb3;
    const float* v;
    int64_t v_nb1, v_nb2, v_nb3;
    int d, n, h, b;
    _Float16* dk;
    _Float16* dv;
};
// The staging as launched: the flat index
// of 8-element groups splits by shifts (d / 8 is a power of two) and
// host-made reciprocals, all 32-bit; K is t = 0, V t = 1.
struct StageArgs {
    const float* src[2];
    int64_t nb1[2], nb2[2], nb3[2];
    _Float16* dst[2];
    uint32_t total8;       // 8-element groups per tensor
    uint32_t c8_log2;      // log2(d / 8)
    DivMod h, n;
};
// Threads of a 256-thread block convert kStageUnits groups each, 256 groups
// apart (2 x kStageUnits 16-byte loads in flight per thread).
constexpr int kStageUnits = 4;
constexpr uint32_t kStageGroupsPerBlock = 256u * kStageUnits;
// Groups [bx * kStageGroupsPerBlock, + kStageGroupsPerBlock) of tensor t,
// converted by thread `tid` of a 256-thread block. NT: nontemporal stores.
template <bool NT>
__device__ __forceinline__ void stage_groups(const StageArgs& sa, uint32_t bx, int t, uint32_t tid) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const uint32_t i0 = bx * kStageGroupsPerBlock + tid;
    f4 x[kStageUnits][2];
#pragma unroll
    for (int u = 0; u < kStageUnits; ++u) {
        const uint32_t i = min(i0 + 256u * u, sa.total8 - 1);   // past the end: reload the last group, store nothing
        const uint32_t r = i >> sa.c8_log2;                     // row index (b, pos, h)
        const uint32_t e = (i - (r << sa.c8_log2)) * 8;         // first element in the row
        const uint32_t r2 = sa.h.div(r);
        const uint32_t hh = r - r2 * sa.h.d;
        const uint32_t bb = sa.n.div(r2);
        const uint32_t pos = r2 - bb * sa.n.d;
        const f4* p = (const f4*)((const char*)sa.src[t] + (int64_t)pos * sa.nb1[t] + (int64_t)hh * sa.nb2[t] +
                                  (int64_t)bb * sa.nb3[t]) + e / 4;
        x[u][0] = __builtin_nontemporal_load(p);
        x[u][1] = __builtin_nontemporal_load(p + 1);
    }
#pragma unroll
    for (int u = 0; u < kStageUnits; ++u) {
        const uint32_t i = i0 + 256u * u;
        h8 y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            y[j] = (_Float16)x[u][0][j];
            y[4 + j] = (_Float16)x[u][1][j];
        }
        if (i < sa.total8) {
            if constexpr (NT) __builtin_nontemporal_store(y, (h8*)(sa.dst[t] + (int64_t)i * 8));
            else *(h8*)(sa.dst[t] + (int64_t)i * 8) = y;
        }
    }
}
// Host: the launch constants of a staging request (false: a shape the
// kernel does not take, d / 8 not a power of two or over 2^31 groups), its
// blocks per tensor, and whether its stores are nontemporal: copies of at
// least 4 MiB (K and V) go past an XCD's L2 anyway, and nontemporal stores
// leave no dirty lines to write back at the end of the launch (encoder F32
// K/V 28.8 -> 28.4 us per layer, realtime encoder 52.7 -> 51.8); a small copy
// (decoder prefill 439, 1.8 MB) keeps ordinary stores, which the next kernel
// finds in L2 (19.8 us against 20.3 with nontemporal stores).
inline bool make_stage_args(const StageReq& r, StageArgs& sa, uint32_t& blocks, bool& nt) {
    if (r.d < 0 || r.d % 8 || (r.d / 8 & (r.d / 8 - 1)) || r.n < 0 || r.h < 0 || r.b < 0) return false;
    const int64_t total8 = (int64_t)r.b * r.n * r.h * (r.d / 8);
    if (total8 > 0x7fffff00) return false;
    blocks = 0;
    nt = false;
    sa.total8 = 0;
    if (total8 == 0) return true;   // nothing to launch
    sa.src[0] = r.k; sa.src[1] = r.v;
    sa.nb1[0] = r.k_nb1; sa.nb2[0] = r.k_nb2; sa.nb3[0] = r.k_nb3;
    sa.nb1[1] = r.v_nb1; sa.nb2[1] = r.v_nb2; sa.nb3[1] = r.v_nb3;
    sa.dst[0] = r.dk; sa.dst[1] = r.dv;
    sa.total8 = (uint32_t)total8;
    uint32_t l2 = 0;
    while ((1 << l2) < r.d / 8) ++l2;
    sa.c8_log2 = l2;
    sa.h = DivMod::make((uint32_t)r.h);
    sa.n = DivMod::make((uint32_t)(r.n > 0 ? r.n : 1));
    blocks = (uint32_t)((total8 + kStageGroupsPerBlock - 1) / kStageGroupsPerBlock);
    nt = (uint64_t)total8 * 32 >= ((uint64_t)4 << 20);
    return true;
}

struct GridMap {
    uint32_t q8, r8;          // nwg / 8, nwg % 8
    uint32_t nqt, hq;
    FastDiv by_nqt, by_hq, by_grp, by_bgrp;   // grp = hq / hkv, bgrp = b / bk
    // Heavy tiles first (hx > 0; masked prefill, where a causal or window
    // mask makes later query tiles longer): XCD x takes the (batch, head)
    // pairs t = b hq + h in [x hx, (x + 1) hx), hx = hq b / 8, and deals its
    // workgroups query tile by query tile from the last: lin / 8 = j gives
    // qt = nqt - 1 - j / hx, t = x hx + j % hx. The heads of one XCD still
    // share its L2, and the first round of workgroups (those dispatched
    // before any ends) holds the longest walks.
    uint32_t hx;
    FastDiv by_hx;
    static GridMap make(int nwg, int nqt, int hq, int hkv, int b, int bk) {
        return GridMap{(uint32_t)nwg >> 3, (uint32_t)nwg & 7, (uint32_t)nqt, (uint32_t)hq,
                       FastDiv::make(nqt), FastDiv::make(hq), FastDiv::make(hq / hkv), FastDiv::make(b / bk),
                       0u, FastDiv::make(1)};
    }
    // the heavy-first order where hq * b is a multiple of 8, else make()'s
    static GridMap make_tiles_desc(int nwg, int nqt, int hq, int hkv, int b, int bk) {
        GridMap g = make(nwg, nqt, hq, hkv, b, bk);
        if ((hq * b) % 8 == 0) {
            g.hx = (uint32_t)(hq * b / 8);
            g.by_hx = FastDiv::make(g.hx);
        }
        return g;
    }
    __host__ __device__ __forceinline__ void locate(uint32_t lin, int& qt, int& h, int& b, int& hk, int& bkv) const {
        const uint32_t xcd = lin & 7;
        uint32_t t;
        if (hx) {
            const uint32_t j = lin >> 3;
            const uint32_t jt = by_hx.div(j);
            qt = (int)(nqt - 1 - jt);
            t = xcd * hx + (j - jt * hx);
        } else {
            const uint32_t gidx = (xcd < r8 ? xcd : r8) * (q8 + 1) + (xcd > r8 ? xcd - r8 : 0u) * q8 + (lin >> 3);
            t = by_nqt.div(gidx);
            qt = (int)(gidx - t * nqt);
        }
        const uint32_t bb = by_hq.div(t);
        h = (int)(t - bb * hq);
        b = (int)bb;
        hk = (int)by_grp.div((uint32_t)h);
        bkv = (int)by_bgrp.div(bb);
    }
};

// F32 -> F16 append of new K/V rows into the cache (the ggml_cpy of
// src/voxtral.cpp:1758-1770 into an f16 cache).
struct AppendArgs {
    const float* k_new;   // [Hkv * D] per token row, rows kn_nb1 apart, batches kn_nb3 apart
    const float* v_new;
    int64_t kn_nb1, kn_nb3, vn_nb1, vn_nb3;
    _Float16* k;          // cache views [D, n_kv, Hkv, Bk] (byte strides)
    _Float16* v;
    int64_t k_nb1, k_nb2, k_nb3, v_nb1, v_nb2, v_nb3;
    int32_t d, hkv, n_new, pos0, bk;   // rows pos0 .. pos0 + n_new - 1 are written
    // K rows rotated first (mode 0) at position rope_pos[b * n_new + t]; null = none
    const int32_t* rope_pos;
    float rope_ts;
    int32_t rope_dims;
};

// Rotary embedding as ggml_rope_ext computes it for mode 0 with
// freq_scale 1, ext_factor 0, attn_factor 1 (the arguments voxtral.cpp
// passes at src/voxtral.cpp:1746-1749 and :1595-1598): pair j = (x[2j],
// x[2j+1]) of a head turns by theta_j, where theta_0 = p and each next
// pair's angle is the previous one times ts = freq_base^(-2 / n_dims), in
// that order (ggml builds its cos/sin cache by this running product), and
// x0' = x0 cos - x1 sin, x1' = x0 sin + x1 cos; dims at or past n_dims are
// left as they are.
//
// (cos, sin) of a float angle: reduced by the nearest multiple q of pi / 2 in
// double precision (error ~1e-12 at the angles rotary embeddings reach), sin
// and cos of the remainder r (|r| <= pi / 4) by their Taylor series through
// r^11 and r^12 (truncation below 1e-11, float rounding a few ulp), then the
// quadrant q mod 4 swaps and negates them. Straight-line code: the library's
// sincosf carries a large-argument path whose code, repeated for every pair a
// lane rotates, cost more than the arithmetic.
__host__ __device__ __forceinline__ float2 rope_cs_of_angle(float th) {
    const double td = (double)th;
    const double qd = __builtin_rint(td * 0.63661977236758134);   // 2 / pi
    const float r = (float)__builtin_fma(-qd, 1.5707963267948966, td);
    const int q = (int)(long long)qd & 3;
    const float r2 = r * r;
    float sn = -2.5052108385e-8f;            // -1/11!
    sn = fmaf(sn, r2, 2.7557319224e-6f);      //  1/9!
    sn = fmaf(sn, r2, -1.9841269841e-4f);     // -1/7!
    sn = fmaf(sn, r2, 8.3333333333e-3f);      //  1/5!
    sn = fmaf(sn, r2, -1.6666666667e-1f);     // -1/3!
    sn = fmaf(sn * r2, r, r);
    float cs = 2.0876756988e-9f;              //  1/12!
    cs = fmaf(cs, r2, -2.7557319224e-7f);     // -1/10!
    cs = fmaf(cs, r2, 2.4801587302e-5f);      //  1/8!
    cs = fmaf(cs, r2, -1.3888888889e-3f);     // -1/6!
    cs = fmaf(cs, r2, 4.1666666667e-2f);      //  1/4!
    cs = fmaf(cs, r2, -0.5f);
    cs = fmaf(cs, r2, 1.0f);
    // angle = q pi / 2 + r: q = 1 gives (-sin r, cos r), 2 (-cos r, -sin r),
    // 3 (sin r, -cos r)
    const float cq = (q & 1) ? sn : cs;
    const float sq = (q & 1) ? cs : sn;
    return float2{(q == 1 || q == 2) ? -cq : cq, (q & 2) ? -sq : sq};
}
// cos / sin of pair j's angle at position p: the running product to pair j
__host__ __device__ __forceinline__ float2 rope_cs(int p, int j, float ts) {
    float th = (float)p;
    for (int i = 0; i < j; ++i) th *= ts;
    return rope_cs_of_angle(th);
}
// rope_cs for pair j < NP of one position p shared by the calling lanes: every
// lane runs the same NP - 1 step running product (fully unrolled, two VALU
// instructions a step) and keeps step j, instead of a loop whose trip count
// differs per lane (~6 instructions an iteration, up to NP - 1 iterations).
template <int NP>
__device__ __forceinline__ float2 rope_cs_chain(int p, int j, float ts) {
    float th = (float)p, mine = th;
#pragma unroll
    for (int i = 1; i < NP; ++i) {
        th *= ts;
        mine = j == i ? th : mine;
    }
    return rope_cs_of_angle(mine);
}

// x holds dims d0 .. d0 + 7 (d0 even), the pairs' cos / sin taken from a table:
// cs[j] = rope_cs(p, j, ts).
__device__ __forceinline__ void rope8_tab(float (&x)[8], int d0, const float2* cs, int n_dims) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (d0 + 2 * k < n_dims) {
            const float2 t = cs[d0 / 2 + k];
            const float x0 = x[2 * k], x1 = x[2 * k + 1];
            x[2 * k] = x0 * t.x - x1 * t.y;
            x[2 * k + 1] = x0 * t.y + x1 * t.x;
        }
    }
}

// x holds dims d0 .. d0 + 7 (d0 even), the four pairs' angles given (pairs
// d0 / 2 .. d0 / 2 + 3)
__device__ __forceinline__ void rope8_ang(float (&x)[8], const float (&ang)[4], int d0, int n_dims) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (d0 + 2 * k < n_dims) {
            const float2 cs = rope_cs_of_angle(ang[k]);
            const float x0 = x[2 * k], x1 = x[2 * k + 1];
            x[2 * k] = x0 * cs.x - x1 * cs.y;
            x[2 * k + 1] = x0 * cs.y + x1 * cs.x;
        }
    }
}

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

// Live range [lo, hi) over `rows` mask rows of n entries each (row r at
// base + r * row_stride bytes): lo is the first and hi - 1 the last column
// holding an entry other than -inf in any of the rows; lo = hi = 0 when every
// entry is -inf. Every thread of the block calls it and gets the result.
// Each row is read as the 16-byte-aligned chunks that cover it, whatever the
// row's alignment: a chunk holds at least one byte of the row, so it lies in
// the same 16-byte granule (same allocation, same page) as mask data, and
// entries outside the row are dropped in registers. A thread takes chunks
// tid, tid + NT, ... eight at a time, all eight loads issued before any is
// tested (a 16K-entry row at 256 threads is one memory round trip). A chunk
// of eight -inf entries is recognised with two word compares; only chunks
// holding a live entry work out its first and last column.
// red: 2 ints of LDS per wavefront.
template <int NT>
__device__ __forceinline__ void mask_live_range(const uint16_t* base, int64_t row_stride, int rows, int n, int* red,
                                                int& lo, int& hi) {
    constexpr int U = 8;
    const int tid = threadIdx.x;
    // chunks per row: exact when every row has the first row's alignment
    const int mis0 = (int)(reinterpret_cast<uintptr_t>(base) & 15);
    const int ncr = (rows == 1 || (row_stride & 15) == 0) ? (mis0 + 2 * n + 15) / 16 : (2 * n + 15) / 16 + 1;
    const int items = rows * ncr;
    constexpr uint32_t DEAD = 0xFC00FC00u;
    int tlo = 0x7fffffff, thi = -1;
    // (one row, the common case: chunk i is column chunk i, no division)
    auto scan = [&](auto one_row) {
        for (int i0 = tid; i0 < items; i0 += U * NT) {
            u32x4 w[U];
            int col[U];   // row column of the chunk's first entry (may be < 0); n when unused
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = i0 + u * NT;
                const int r = decltype(one_row)::value ? 0 : i / ncr, c = i - r * ncr;
                const char* rowp = reinterpret_cast<const char*>(base) + (int64_t)r * row_stride;
                const int off = 16 * c - (int)(reinterpret_cast<uintptr_t>(rowp) & 15);   // bytes from the row start
                const bool ok = i < items && off < 2 * n;
                col[u] = ok ? off / 2 : n;
                w[u] = u32x4{DEAD, DEAD, DEAD, DEAD};
                if (ok) w[u] = *reinterpret_cast<const u32x4*>(rowp + off);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if ((w[u][0] & w[u][1]) == DEAD && (w[u][2] & w[u][3]) == DEAD &&
                    (w[u][0] | w[u][1] | w[u][2] | w[u][3]) == DEAD)
                    continue;   // eight -inf entries
                uint32_t m = 0;   // bit e: entry e is not -inf
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    m |= ((w[u][j] & 0xFFFFu) != kF16NegInf ? 1u : 0u) << (2 * j);
                    m |= ((w[u][j] >> 16) != kF16NegInf ? 1u : 0u) << (2 * j + 1);
                }
                if (col[u] < 0 || col[u] > n - 8) {   // a chunk reaching outside the row
                    const int e_lo = min(max(-col[u], 0), 8), e_hi = min(max(n - col[u], 0), 8);
                    m &= e_hi > e_lo ? ((1u << (e_hi - e_lo)) - 1u) << e_lo : 0u;
                }
                if (m) {
                    tlo = min(tlo, col[u] + (int)__builtin_ctz(m));
                    thi = max(thi, col[u] + 31 - (int)__builtin_clz(m));
                }
            }
        }
    };
    if (rows == 1) scan(std::true_type{});
    else scan(std::false_type{});
    // wavefront min / max: DPP row rotations, then the lane pairs 16 and 32
    // apart (VALU lane swaps; no LDS round trips on the way to the range)
    auto rot_min_max = [&](auto ctl) {   // DPP row_ror by ctl - 0x120
        constexpr int C = decltype(ctl)::value;
        tlo = min(tlo, __builtin_amdgcn_update_dpp(0, tlo, C, 0xF, 0xF, false));
        thi = max(thi, __builtin_amdgcn_update_dpp(0, thi, C, 0xF, 0xF, false));
    };
    rot_min_max(std::integral_constant<int, 0x128>{});
    rot_min_max(std::integral_constant<int, 0x124>{});
    rot_min_max(std::integral_constant<int, 0x122>{});
    rot_min_max(std::integral_constant<int, 0x121>{});
    {
        const auto l16 = __builtin_amdgcn_permlane16_swap(tlo, tlo, false, false);
        const auto h16 = __builtin_amdgcn_permlane16_swap(thi, thi, false, false);
        tlo = min((int)l16[0], (int)l16[1]);
        thi = max((int)h16[0], (int)h16[1]);
        const auto l32 = __builtin_amdgcn_permlane32_swap(tlo, tlo, false, false);
        const auto h32 = __builtin_amdgcn_permlane32_swap(thi, thi, false, false);
        tlo = min((int)l32[0], (int)l32[1]);
        thi = max((int)h32[0], (int)h32[1]);
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
constexpr int kDecodeMaxSplit = 64;  // split workgroups per (batch, kv head)
constexpr int kDecodeWaves = 4;      // wavefronts per decode workgroup
// Floats per decode partial record: O [G][D], then m [G] and l [G], padded to
// a multiple of 4 so every record starts 16-byte aligned.
constexpr int dec_record_floats(int D, int G) { return G * D + ((2 * G + 3) & ~3); }
hipError_t launch_prefill(const AttnArgs& a, int head_dim, int waves, hipStream_t stream);
// hd 64 prefill on the pipelined kernel: no mask, an implicit mask, or a mask
// tensor (a.mask_rows: workspace for nq * hm * bm intervals, filled first by
// a pre-pass launch)
// stage: F32 K/V to convert first (a.k / a.v already point at the f16
// copies), or null; with a mask tensor the conversion and the pre-pass share
// one launch
hipError_t launch_prefill64_pp(const AttnArgs& a, const StageReq* stage, hipStream_t stream);
// the mask pre-pass: the live interval of each of the nq * hm * bm rows of
// a.mask into a.mask_rows, in one launch with the F32 -> f16 staging of
// *stage when stage is not null
hipError_t launch_mask_prep(const AttnArgs& a, const StageReq* stage, hipStream_t stream);
// masked hd 128 prefill with n_kv <= 512 (a mask tensor or an implicit mask;
// a rotary embedding of F32 Q); with a mask tensor and a.mask_rows set the
// intervals there (launch_mask_prep first) give the block classes
hipError_t launch_prefill_pair(const AttnArgs& a, hipStream_t stream);
// whether launch_prefill_pair takes these strides (its 32-bit offsets)
bool prefill_pair_fits(const AttnArgs& a);
hipError_t launch_zero(float* dst, int64_t n, hipStream_t stream);
hipError_t launch_kv_append(const AppendArgs& a, hipStream_t stream);
// F32 -> f16 copies of K and V (StageReq above), one launch of their own
hipError_t launch_to_f16_kv(const StageReq& r, hipStream_t stream);
}  // namespace vxfa
