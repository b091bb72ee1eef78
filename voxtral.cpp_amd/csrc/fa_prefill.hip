// fa_prefill.hip — multi-query attention (prefill) for gfx950 with f16 MFMA.
//
// Replaces the backend kernel of GGML_OP_FLASH_ATTN_EXT for the prefill
// calls voxtral.cpp makes:
//   encoder self-attention, hd 64, no mask offline    (src/voxtral.cpp:1611)
//   decoder prefill, GQA 32/8, hd 128, causal mask     (src/voxtral.cpp:1802,
//       mask built by fill_causal_mask :2104-2111)
//
// Work decomposition
//   One workgroup per (block of BM = 32 * NQW query rows, query head, batch)
//   with NQW * KVG wavefronts: wavefront (qw, kg) owns query rows
//   [32 qw, 32 qw + 32) of the block and the kg-th 64-position half of every
//   128-position KV step (KVG = 2). The two KV halves give each SIMD two
//   independent wavefronts, so one's softmax (VALU) runs beside the other's
//   MFMAs; they are merged through LDS at the end.
//   The 1-D grid is mapped so the workgroups that share one head's K/V are
//   dispatched to the same XCD (workgroups are dealt to the 8 XCDs round
//   robin), keeping that head's K/V in one L2. Without a mask each workgroup
//   starts its KV walk at an offset set by its query block, so the workgroups
//   of one head do not all miss on the same tile at once.
// Pipeline: K/V steps are double buffered in LDS; the step after next is in
//   flight in registers; one barrier per step.
// MFMA layouts (v_mfma_f32_32x32x16_f16, lane = 32*hh + nl):
//   S^T = K Q^T: A = K rows from LDS (128-bit reads), B = Q (registers, f16
//     rounded like ggml's Q conversion). Lane (nl, hh) receives query row nl
//     and 16 contiguous KV positions of each 32-block, so the row max needs
//     one cross-lane step (v_permlane32_swap).
//   O^T = V^T P^T: B = P straight from the softmax registers (f16), A = V^T
//     fetched from the row-major V tile with ds_read_b64_tr_b16, which
//     transposes 16-bit elements across each 16-lane group.
// Softmax in fp32 with exp2 (scale*log2(e) folded into one FMA per score).
//   The running max is raised only when a tile's max exceeds it by more than
//   2^8, so the O rescale runs on few tiles; P then stays below 256 in f16.
// Row-to-KV mapping inside a 32-position block (lane half hh, accumulator
// element j, a = j / 4, b = j % 4):
//   hh = 0 : kv = 4a + b            hh = 1 : kv = 16 + 4((a + 2) & 3) + b
// so that (1) the K rows one 16-lane LDS phase reads fall in 16 distinct
// bank groups with a 16-byte row padding, and (2) each half of a lane's
// accumulator (j < 8, j >= 8) covers 8 contiguous positions in increasing
// order, the order the P.V operand needs.
#include "fa_common.h"

#include <type_traits>

namespace vxfa {

constexpr int PF_BN = 64;                // KV positions per wavefront tile
constexpr float PF_TAU = 8.0f;
constexpr int PF_MAX_TILE_WORDS = 256;   // live-tile bitmap: up to 8192 tiles

typedef short short4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int pf_kv_of(int hh, int j) {
    return hh ? 16 + (((j >> 2) + 2) & 3) * 4 + (j & 3) : j;
}

// Four 16-bit elements, transposed across each 16-lane group: lane i of the
// group receives element (i % 4) of the 8 bytes addressed by lane 4r + i/4,
// for r = 0..3 (gfx950 ds_read_b64_tr_b16).
__device__ __forceinline__ half4 lds_read_tr16(const _Float16* p) {
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(p));
    return __builtin_bit_cast(half4, r);
}

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

template <int D, int NQW, int KVG, bool MASK, bool QF16>
__global__ __launch_bounds__(64 * NQW * KVG) void fa_prefill_kernel(AttnArgs a, int nqt) {
    static_assert(D == 64 || D == 128, "head dim");
    static_assert(KVG == 1 || KVG == 2, "kv groups");
    constexpr int NT = 64 * NQW * KVG;
    constexpr int BM = 32 * NQW;
    constexpr int BS = PF_BN * KVG;    // KV positions per step
    constexpr int KSTR = D + 8;        // halfs per K row in LDS: odd number of 16-byte units
    constexpr int VSTR = D + 16;       // halfs per V row in LDS: the 4 rows of a tr-read hit distinct banks
    constexpr int KS = D / 16;         // S-MFMA k-steps
    constexpr int DB = D / 32;         // O^T row blocks
    constexpr int CH = D / 8;          // 16-byte chunks per row
    constexpr int NCH = BS * CH / NT;  // chunks per thread per step (K and V each)
    static_assert(NCH * NT == BS * CH, "step split");
    constexpr int KBYTES = BS * KSTR * 2, VBYTES = BS * VSTR * 2;

    __shared__ __attribute__((aligned(16))) char smem[2 * (KBYTES + VBYTES)];
    __shared__ uint32_t s_live[MASK ? PF_MAX_TILE_WORDS : 1];
    auto sK = [&](int st) { return (_Float16*)(smem + st * (KBYTES + VBYTES)); };
    auto sV = [&](int st) { return (_Float16*)(smem + st * (KBYTES + VBYTES) + KBYTES); };

    // ---- XCD-aware position of this workgroup --------------------------------
    const int nwg = gridDim.x;
    const int lin = blockIdx.x;
    const int xcd = lin & 7, q8 = nwg >> 3, r8 = nwg & 7;
    const int gidx = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + (lin >> 3);
    const int qt = gidx % nqt;
    const int h = (gidx / nqt) % a.hq;
    const int b = gidx / (nqt * a.hq);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int qw = wave % NQW;
    const int kg = wave / NQW;
    const int q0 = qt * BM;
    const int hk = h / (a.hq / a.hkv);
    const int bkv = b / (a.b / a.bk);
    const char* kb = (const char*)a.k + (int64_t)hk * a.k_nb2 + (int64_t)bkv * a.k_nb3;
    const char* vb = (const char*)a.v + (int64_t)hk * a.v_nb2 + (int64_t)bkv * a.v_nb3;

    const int nl = lane & 31;
    const int hh = lane >> 5;
    const int qrow = q0 + qw * 32 + nl;
    const bool qvalid = qrow < a.nq;
    const int ntile = (a.nkv + PF_BN - 1) / PF_BN;   // 64-position tiles
    const int nstep = (a.nkv + BS - 1) / BS;         // BS-position steps

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
                const uint16_t* mr = (const uint16_t*)((const char*)mplane + (int64_t)(q0 + r) * a.m_nb1);
                for (int cc = tid; cc < a.nkv; cc += NT) {
                    if (mr[cc] != kF16NegInf) {
                        const int tile = cc / PF_BN;
                        const uint32_t bit = 1u << (tile & 31);
                        if (!(s_live[tile >> 5] & bit)) atomicOr(&s_live[tile >> 5], bit);
                    }
                }
            }
            __syncthreads();
        }
    }
    // Step sequence: without a mask all steps, rotated by the query block;
    // with a mask the steps holding a live tile, in order. -1 ends it.
    const bool seq_all = !MASK || !use_bitmap;
    const int rot = MASK ? 0 : (int)(((int64_t)qt * nstep) / nqt) % nstep;
    auto step_live = [&](int s) -> bool {
        bool live = false;
#pragma unroll
        for (int g = 0; g < KVG; ++g) {
            const int t = s * KVG + g;
            if (t < ntile && ((s_live[t >> 5] >> (t & 31)) & 1u)) live = true;
        }
        return live;
    };
    auto advance = [&](int s) -> int {
        if (s < 0) return -1;
        if (seq_all) {
            const int idx = (s - rot + nstep) % nstep + 1;
            return idx < nstep ? (rot + idx) % nstep : -1;
        }
        for (int u = s + 1; u < nstep; ++u)
            if (step_live(u)) return u;
        return -1;
    };
    int first = -1;
    if (seq_all) {
        first = rot;
    } else {
        for (int u = 0; u < nstep; ++u)
            if (step_live(u)) { first = u; break; }
    }

    // ---- Q operand (B of S^T = K Q^T): row qrow, dims 16ks + 8hh .. +7 ----
    // (the Q element type is a template parameter: a load-or-convert branch on
    // it makes the compiler wait for all global loads inside the KV loop)
    half8 qb[KS];
    {
        constexpr int qelt = QF16 ? 2 : 4;
        const int64_t qoff = (int64_t)(qvalid ? qrow : 0) * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (qvalid) qb[ks] = load_q8(a.q, qoff + (int64_t)(16 * ks + 8 * hh) * qelt, QF16);
            else qb[ks] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    // ---- step staging: global -> registers -> LDS (row-major K and V) -------
    half8 rk[NCH], rv[NCH];
    auto gload = [&](int s) {
        const int kv0 = s * BS;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int ci = tid + i * NT;
            const int kv = min(kv0 + ci / CH, a.nkv - 1);
            rk[i] = *(const half8*)(kb + (int64_t)kv * a.k_nb1 + (ci % CH) * 16);
            rv[i] = *(const half8*)(vb + (int64_t)kv * a.v_nb1 + (ci % CH) * 16);
        }
    };
    auto swrite = [&](int st) {
        _Float16* k = sK(st);
        _Float16* v = sV(st);
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int ci = tid + i * NT;
            *(half8*)&k[(ci / CH) * KSTR + (ci % CH) * 8] = rk[i];
            *(half8*)&v[(ci / CH) * VSTR + (ci % CH) * 8] = rv[i];
        }
    };

    floatx16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    // K row fetched by this lane as A-operand row nl of each 32-block (within
    // this wavefront's 64-position tile of the step)
    int krow0;
    {
        const int am = nl >> 3, ahb = (nl >> 2) & 1, ab = nl & 3;
        krow0 = PF_BN * kg + (ahb ? 16 + ((am + 2) & 3) * 4 + ab : 4 * am + ab);
    }
    // lane's element offset inside the V tile for the transposed reads: row
    // (lane % 16) / 4 of a 4-row group, dims 16 * ((lane % 32) / 16) + 4 * (lane % 4)
    const int v_lane_off = (PF_BN * kg + ((lane & 15) >> 2)) * VSTR + 16 * ((lane & 31) >> 4) + 4 * (lane & 3);
    const uint16_t* mrow = nullptr;
    if (MASK) mrow = (const uint16_t*)((const char*)mplane + (int64_t)(qvalid ? qrow : 0) * a.m_nb1);
    const half2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    const float c = a.scale_log2;

    // one 64-position tile at kv0 from LDS stage st.
    // TAIL: the tile runs past n_kv (positions >= n_kv are forced to -inf).
    auto tile = [&](auto tail_tag, int st, int kv0) {
        constexpr bool TAIL = decltype(tail_tag)::value;
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
        if (!live) return;

        // hd 64: every LDS operand of the tile is requested up front, so the
        // V^T reads complete behind the S MFMAs and the softmax instead of
        // stalling P.V (hd 128 has no registers to spare and reads V^T late).
        constexpr bool HOIST = (D == 64);
        const _Float16* ks_ = sK(st);
        const _Float16* vs = sV(st) + v_lane_off;
        auto read_va = [&](int pc, int db) -> half8 {
            // the 8 positions of operand pc, increasing from kvl
            const int kvl = 32 * (pc >> 1) + (hh ? 16 + 8 * (1 - (pc & 1)) : 8 * (pc & 1));
            const _Float16* p = vs + kvl * VSTR + 32 * db;
            const half4 lo4 = lds_read_tr16(p);
            const half4 hi4 = lds_read_tr16(p + 4 * VSTR);
            return half8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        };
        half8 ka[2][KS];
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                ka[kvb][ks] = *(const half8*)&ks_[(32 * kvb + krow0) * KSTR + 16 * ks + 8 * hh];
        half8 va[HOIST ? 4 : 1][DB];
        if constexpr (HOIST) {
#pragma unroll
            for (int pc = 0; pc < 4; ++pc)
#pragma unroll
                for (int db = 0; db < DB; ++db) va[pc][db] = read_va(pc, db);
        }
        floatx16 S[2];
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb) {
#pragma unroll
            for (int j = 0; j < 16; ++j) S[kvb][j] = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                S[kvb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[kvb][ks], qb[ks], S[kvb], 0, 0, 0);
        }

        // Row max in log2 units. Without a mask the scale is applied after the
        // max (max(c*s) = c*max(s) for c >= 0, c*min(s) for c < 0) and folded
        // into the exp2 argument, one FMA per score.
        float mx;
        if (MASK || TAIL) {
            mx = -INFINITY;
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    float x = S[kvb][j] * c;
                    if (MASK) x = (mv[kvb][j] == -INFINITY) ? -INFINITY : x + mv[kvb][j];
                    if (TAIL && kv0 + 32 * kvb + pf_kv_of(hh, j) >= a.nkv) x = -INFINITY;
                    S[kvb][j] = x;
                    mx = fmaxf(mx, x);
                }
        } else if (c >= 0.f) {
            float r = S[0][0];
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int j = 0; j < 16; ++j) r = fmaxf(r, S[kvb][j]);
            mx = r * c;
        } else {
            float r = S[0][0];
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int j = 0; j < 16; ++j) r = fminf(r, S[kvb][j]);
            mx = r * c;
        }
        mx = pair32_max(mx);

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

        float lsum[2] = {0.f, 0.f};
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {
            const int kvb = pc >> 1, cc = pc & 1;
            half8 pb;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float e = (MASK || TAIL) ? S[kvb][8 * cc + i] - msafe : fmaf(S[kvb][8 * cc + i], c, -msafe);
                pb[i] = (_Float16)exp2_fast(e);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                half2 p2 = {pb[2 * i], pb[2 * i + 1]};
                lsum[i & 1] = __builtin_amdgcn_fdot2(p2, ones, lsum[i & 1], false);
            }
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const half8 vop = HOIST ? va[HOIST ? pc : 0][db] : read_va(pc, db);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pb, o[db], 0, 0, 0);
            }
        }
        l_run += lsum[0] + lsum[1];
    };

    // ---- main loop: step s in stage st; step s_next staged at the top of the
    // iteration; step s_next2 in flight in registers -----------------------------
    int s_cur = first;
    int s_nxt = advance(s_cur);
    int s_nx2 = advance(s_nxt);
    if (s_cur >= 0) { gload(s_cur); swrite(0); }
    if (s_nxt >= 0) gload(s_nxt);
    __syncthreads();
    int st = 0;
    while (s_cur >= 0) {
        // the other stage was last read in the previous iteration, before its barrier
        if (s_nxt >= 0) swrite(st ^ 1);
        if (s_nx2 >= 0) gload(s_nx2);
        const int kv0 = s_cur * BS + PF_BN * kg;
        if (kv0 < a.nkv) {
            if (kv0 + PF_BN > a.nkv) tile(std::true_type{}, st, kv0);
            else tile(std::false_type{}, st, kv0);
        }
        __syncthreads();
        s_cur = s_nxt;
        s_nxt = s_nx2;
        s_nx2 = advance(s_nx2);
        st ^= 1;
    }

    // ---- merge the KV groups (LDS), normalise, store dst[b][qrow][h][d] ------
    if (KVG == 2) {
        // group 1 publishes (m, l, O); every staging buffer is free after the
        // loop's last barrier
        float* xo = (float*)smem;                          // [NQW][64 lanes][16 * DB]
        float* xm = xo + NQW * 64 * 16 * DB;               // [NQW][64]
        float* xl = xm + NQW * 64;
        if (kg == 1) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 16; ++j) xo[(qw * 64 + lane) * 16 * DB + db * 16 + j] = o[db][j];
            xm[qw * 64 + lane] = m_run;
            xl[qw * 64 + lane] = l_run;
        }
        __syncthreads();
        if (kg == 1) return;
        const float m2 = xm[qw * 64 + lane], l2 = xl[qw * 64 + lane];
        const float M = fmaxf(m_run, m2);
        const float Ms = (M == -INFINITY) ? 0.f : M;
        const float w1 = exp2_fast(m_run - Ms), w2 = exp2_fast(m2 - Ms);
        l_run = l_run * w1 + l2 * w2;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                o[db][j] = o[db][j] * w1 + xo[(qw * 64 + lane) * 16 * DB + db * 16 + j] * w2;
    }
    const float lt = pair32_sum(l_run);
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

template <int D, int NQW, int KVG>
static hipError_t launch_pw(const AttnArgs& a, hipStream_t st) {
    constexpr int BM = 32 * NQW;
    const int nqt = (a.nq + BM - 1) / BM;
    const int64_t nwg = (int64_t)nqt * a.hq * a.b;
    if (nwg <= 0 || nwg > 0x7fffffff) return hipErrorInvalidValue;
    constexpr int NT = 64 * NQW * KVG;
    const dim3 grid((unsigned)nwg), block(NT);
    if (a.mask) {
        if (a.q_f16) hipLaunchKernelGGL((fa_prefill_kernel<D, NQW, KVG, true, true>), grid, block, 0, st, a, nqt);
        else hipLaunchKernelGGL((fa_prefill_kernel<D, NQW, KVG, true, false>), grid, block, 0, st, a, nqt);
    } else {
        if (a.q_f16) hipLaunchKernelGGL((fa_prefill_kernel<D, NQW, KVG, false, true>), grid, block, 0, st, a, nqt);
        else hipLaunchKernelGGL((fa_prefill_kernel<D, NQW, KVG, false, false>), grid, block, 0, st, a, nqt);
    }
    return hipGetLastError();
}

// waves = query-row wavefronts per workgroup (32 rows each); each has a
// partner wavefront for the second KV half.
hipError_t launch_prefill(const AttnArgs& a, int head_dim, int waves, hipStream_t st) {
    if (head_dim == 64) {
        if (waves == 4) return launch_pw<64, 4, 2>(a, st);
        if (waves == 2) return launch_pw<64, 2, 2>(a, st);
    } else if (head_dim == 128) {
        if (waves == 4) return launch_pw<128, 4, 2>(a, st);
        if (waves == 2) return launch_pw<128, 2, 2>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace vxfa
