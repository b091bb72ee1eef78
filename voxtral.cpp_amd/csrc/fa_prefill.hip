// fa_prefill.hip — multi-query attention (prefill) for gfx950 with f16 MFMA.
//
// Replaces the backend kernel of GGML_OP_FLASH_ATTN_EXT for the prefill
// calls voxtral.cpp makes:
//   encoder self-attention, hd 64, no mask offline    (src/voxtral.cpp:1611)
//   decoder prefill, GQA 32/8, hd 128, causal mask     (src/voxtral.cpp:1802,
//       mask built by fill_causal_mask :2104-2111)
//
// Work decomposition
//   grid  = (ceil(Nq / BM), Hq, B); BM = 32 query rows per wavefront.
//   K/V tiles of 64 positions are staged in LDS (double buffered) and shared
//   by the workgroup's wavefronts; the next tile's global loads are in
//   flight while the current one is computed.
//   S^T = K Q^T with v_mfma_f32_32x32x16_f16: each lane ends up owning one
//   query row (lane & 31) and 16 contiguous KV positions of a 32-block, so
//   the row max needs a single cross-lane step (lane ^ 32).
//   O^T = V^T P^T with the same instruction: P stays in registers (f16), V is
//   written to LDS transposed so each A-operand fetch is one 128-bit read.
//   Softmax in fp32 with exp2 (scale*log2(e) folded in). The running max is
//   only raised when a tile's max exceeds it by more than 2^8, so the O
//   rescale runs on few tiles; P then stays below 256, safe in f16.
// Row-to-KV mapping inside a 32-position block (lane half hh, element j of
// the MFMA accumulator, a = j / 4, b = j % 4):
//   hh = 0 : kv = 4a + b            hh = 1 : kv = 16 + 4((a + 2) & 3) + b
// chosen so that (1) the K rows one 16-lane LDS phase reads fall in 16
// distinct bank groups with a 16-byte row padding, and (2) each half of a
// lane's accumulator (j < 8, j >= 8) covers 8 contiguous positions in
// increasing order, so P feeds the P.V MFMA without any register permutation
// and V^T is fetched with one 128-bit read.
#include "fa_common.h"

#include <type_traits>

namespace vxfa {

constexpr int PF_BN = 64;
constexpr float PF_TAU = 8.0f;
constexpr int PF_MAX_TILE_WORDS = 256;   // live-tile bitmap: up to 8192 tiles

__device__ __forceinline__ int pf_kv_of(int hh, int j) {
    return hh ? 16 + (((j >> 2) + 2) & 3) * 4 + (j & 3) : j;
}

template <int D, int NW, bool MASK>
__global__ __launch_bounds__(64 * NW) void fa_prefill_kernel(AttnArgs a) {
    static_assert(D == 64 || D == 128, "head dim");
    constexpr int NT = 64 * NW;
    constexpr int BM = 32 * NW;
    constexpr int KSTR = D + 8;        // halfs per K row in LDS
    constexpr int VSTR = PF_BN + 8;    // halfs per V^T row in LDS
    constexpr int KS = D / 16;         // S-MFMA k-steps
    constexpr int DB = D / 32;         // O^T row blocks
    constexpr int KCH = D / 8;         // 16-byte chunks per row
    constexpr int K_IT = PF_BN * KCH / NT;
    constexpr int V_IT = (PF_BN / 2) * KCH / NT;
    static_assert(K_IT * NT == PF_BN * KCH, "K tile split");
    static_assert(V_IT * NT == (PF_BN / 2) * KCH, "V tile split");

    __shared__ __attribute__((aligned(16))) _Float16 sK[2][PF_BN * KSTR];
    __shared__ __attribute__((aligned(16))) _Float16 sVT[2][D * VSTR];
    __shared__ uint32_t s_live[MASK ? PF_MAX_TILE_WORDS : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int q0 = blockIdx.x * BM;
    const int hk = h / (a.hq / a.hkv);
    const int bkv = b / (a.b / a.bk);
    const char* kb = (const char*)a.k + (int64_t)hk * a.k_nb2 + (int64_t)bkv * a.k_nb3;
    const char* vb = (const char*)a.v + (int64_t)hk * a.v_nb2 + (int64_t)bkv * a.v_nb3;

    const int nl = lane & 31;
    const int hh = lane >> 5;
    const int qrow = q0 + wave * 32 + nl;
    const bool qvalid = qrow < a.nq;
    const int ntile = (a.nkv + PF_BN - 1) / PF_BN;

    // ---- Q operand (B of S^T = K Q^T): row qrow, dims 16ks + 8hh .. +7 ----
    half8 qb[KS];
    {
        const int qelt = a.q_f16 ? 2 : 4;
        const int64_t qoff = (int64_t)(qvalid ? qrow : 0) * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (qvalid) qb[ks] = load_q8(a.q, qoff + (int64_t)(16 * ks + 8 * hh) * qelt, a.q_f16 != 0);
            else qb[ks] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    // ---- live tiles of the mask for this workgroup's rows -----------------
    const uint16_t* mplane = nullptr;
    bool use_bitmap = false;
    if (MASK) {
        mplane = (const uint16_t*)((const char*)a.mask + (int64_t)(h % a.hm) * a.m_nb2 +
                                   (int64_t)(b % a.bm) * a.m_nb3);
        const int words = (ntile + 31) / 32;
        use_bitmap = words <= PF_MAX_TILE_WORDS;
        if (use_bitmap) {
            for (int i = tid; i < words; i += NT) s_live[i] = 0u;
            __syncthreads();
            const int rows = min(BM, a.nq - q0);
            for (int r = 0; r < rows; ++r) {
                const uint16_t* mrow = (const uint16_t*)((const char*)mplane + (int64_t)(q0 + r) * a.m_nb1);
                for (int c = tid; c < a.nkv; c += NT) {
                    if (mrow[c] != kF16NegInf) {
                        const int tile = c / PF_BN;
                        const uint32_t bit = 1u << (tile & 31);
                        if (!(s_live[tile >> 5] & bit)) atomicOr(&s_live[tile >> 5], bit);
                    }
                }
            }
            __syncthreads();
        }
    }
    auto next_tile = [&](int t) -> int {
        if (!MASK || !use_bitmap) return t;
        while (t < ntile) {
            const uint32_t w = s_live[t >> 5] >> (t & 31);
            if (w) return t + __builtin_ctz(w);
            t = (t | 31) + 1;
        }
        return ntile;
    };

    // ---- tile staging -------------------------------------------------------
    half8 kreg[K_IT];
    half8 vreg[V_IT][2];
    auto gload = [&](int t) {
        const int kv0 = t * PF_BN;
#pragma unroll
        for (int i = 0; i < K_IT; ++i) {
            const int c = tid + i * NT;
            const int kv = min(kv0 + c / KCH, a.nkv - 1);
            kreg[i] = *(const half8*)(kb + (int64_t)kv * a.k_nb1 + (c % KCH) * 16);
        }
#pragma unroll
        for (int i = 0; i < V_IT; ++i) {
            const int u = tid + i * NT;
            const int pr = u & 31, ch = u >> 5;
            const int kva = min(kv0 + 2 * pr, a.nkv - 1);
            const int kvb2 = min(kv0 + 2 * pr + 1, a.nkv - 1);
            vreg[i][0] = *(const half8*)(vb + (int64_t)kva * a.v_nb1 + ch * 16);
            vreg[i][1] = *(const half8*)(vb + (int64_t)kvb2 * a.v_nb1 + ch * 16);
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < K_IT; ++i) {
            const int c = tid + i * NT;
            *(half8*)&sK[buf][(c / KCH) * KSTR + (c % KCH) * 8] = kreg[i];
        }
#pragma unroll
        for (int i = 0; i < V_IT; ++i) {
            const int u = tid + i * NT;
            const int pr = u & 31, ch = u >> 5;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                half2 pk = {vreg[i][0][e], vreg[i][1][e]};
                *(half2*)&sVT[buf][(ch * 8 + e) * VSTR + 2 * pr] = pk;
            }
        }
    };

    floatx16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    // K row (within the tile) fetched by this lane as A-operand row nl
    int krow[2];
    {
        const int am = nl >> 3, ahb = (nl >> 2) & 1, ab = nl & 3;
        const int kv = ahb ? 16 + ((am + 2) & 3) * 4 + ab : 4 * am + ab;
        krow[0] = kv;
        krow[1] = 32 + kv;
    }
    const uint16_t* mrow = nullptr;
    if (MASK) mrow = (const uint16_t*)((const char*)mplane + (int64_t)(qvalid ? qrow : 0) * a.m_nb1);
    const half2 ones = {(_Float16)1.0f, (_Float16)1.0f};

    const float c = a.scale_log2;

    // One KV tile for this wavefront. TAIL: the tile runs past n_kv, so
    // positions >= n_kv are forced to -inf (only the last tile can be).
    auto tile_body = [&](auto tail_tag, int buf, int kv0) {
        constexpr bool TAIL = decltype(tail_tag)::value;

        // mask values for this lane's 32 scores
        float mv[2][16];
        bool live = true;
        if (MASK) {
            bool any = false;
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int kv = kv0 + 32 * kvb + pf_kv_of(hh, j);
                    float m = -INFINITY;
                    if (qvalid && kv < a.nkv) m = f16_bits_to_f32(mrow[kv]);
                    mv[kvb][j] = m * kLog2e;
                    any |= (m != -INFINITY);
                }
            live = __any(any);
        }

        if (live) {
            floatx16 st[2];
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb) {
#pragma unroll
                for (int j = 0; j < 16; ++j) st[kvb][j] = 0.f;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const half8 ka = *(const half8*)&sK[buf][krow[kvb] * KSTR + 16 * ks + 8 * hh];
                    st[kvb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb[ks], st[kvb], 0, 0, 0);
                }
            }

            // Row max in log2 units. Without a mask the scale is applied after
            // the max (max(c*s) = c*max(s) for c >= 0, c*min(s) for c < 0) and
            // folded into the exp2 argument below, one FMA per score.
            float mx;
            if (MASK || TAIL) {
                mx = -INFINITY;
#pragma unroll
                for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        float x = st[kvb][j] * c;
                        if (MASK) x = (mv[kvb][j] == -INFINITY) ? -INFINITY : x + mv[kvb][j];
                        if (TAIL && kv0 + 32 * kvb + pf_kv_of(hh, j) >= a.nkv) x = -INFINITY;
                        st[kvb][j] = x;
                        mx = fmaxf(mx, x);
                    }
            } else if (c >= 0.f) {
                float r = st[0][0];
#pragma unroll
                for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                    for (int j = 0; j < 16; ++j) r = fmaxf(r, st[kvb][j]);
                mx = r * c;
            } else {
                float r = st[0][0];
#pragma unroll
                for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                    for (int j = 0; j < 16; ++j) r = fminf(r, st[kvb][j]);
                mx = r * c;
            }
            mx = fmaxf(mx, shfl_xor(mx, 32));

            if (__any(mx > m_run + PF_TAU)) {
                const float mnew = fmaxf(m_run, mx);
                const float ms = (mnew == -INFINITY) ? 0.f : mnew;
                const float alpha = exp2_fast(m_run - ms);
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int j = 0; j < 16; ++j) o[db][j] *= alpha;
                l_run *= alpha;
                m_run = mnew;
            }
            const float msafe = (m_run == -INFINITY) ? 0.f : m_run;

#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int kvb = c >> 1, cc = c & 1;
                half8 pb;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float e = (MASK || TAIL) ? st[kvb][8 * cc + i] - msafe
                                                   : fmaf(st[kvb][8 * cc + i], c, -msafe);
                    pb[i] = (_Float16)exp2_fast(e);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    half2 p2 = {pb[2 * i], pb[2 * i + 1]};
                    l_run = __builtin_amdgcn_fdot2(p2, ones, l_run, false);
                }
                const int kvl = 32 * kvb + (hh ? 16 + 8 * (1 - cc) : 8 * cc);  // 8 positions, increasing
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const half8 va = *(const half8*)&sVT[buf][(32 * db + nl) * VSTR + kvl];
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[db], 0, 0, 0);
                }
            }
        }
    };

    int t = next_tile(0);
    if (t < ntile) gload(t);
    int buf = 0;
    while (t < ntile) {
        swrite(buf);
        __syncthreads();
        const int tn = next_tile(t + 1);
        if (tn < ntile) gload(tn);
        const int kv0 = t * PF_BN;
        if (kv0 + PF_BN > a.nkv) tile_body(std::true_type{}, buf, kv0);
        else tile_body(std::false_type{}, buf, kv0);
        buf ^= 1;
        t = tn;
    }

    // ---- normalise and store: dst[b][qrow][h][d] ----------------------------
    const float lt = l_run + shfl_xor(l_run, 32);
    const float inv = (lt == 0.f) ? 0.f : 1.0f / lt;
    if (qvalid) {
        float* out = a.dst + (((int64_t)b * a.nq + qrow) * a.hq + h) * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int d0 = 32 * db + 8 * a4 + 4 * hh;
                floatx4 vv = {o[db][4 * a4] * inv, o[db][4 * a4 + 1] * inv, o[db][4 * a4 + 2] * inv,
                              o[db][4 * a4 + 3] * inv};
                *(floatx4*)(out + d0) = vv;
            }
    }
}

template <int D, int NW>
static hipError_t launch_pw(const AttnArgs& a, hipStream_t st) {
    constexpr int BM = 32 * NW;
    dim3 grid((a.nq + BM - 1) / BM, a.hq, a.b);
    if (a.mask)
        hipLaunchKernelGGL((fa_prefill_kernel<D, NW, true>), grid, dim3(64 * NW), 0, st, a);
    else
        hipLaunchKernelGGL((fa_prefill_kernel<D, NW, false>), grid, dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_prefill(const AttnArgs& a, int head_dim, int waves, hipStream_t st) {
    if (head_dim == 64) {
        if (waves == 4) return launch_pw<64, 4>(a, st);
        if (waves == 2) return launch_pw<64, 2>(a, st);
    } else if (head_dim == 128) {
        if (waves == 4) return launch_pw<128, 4>(a, st);
        if (waves == 2) return launch_pw<128, 2>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace vxfa
