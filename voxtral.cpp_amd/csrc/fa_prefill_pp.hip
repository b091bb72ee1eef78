// fa_prefill_pp.hip — encoder self-attention prefill (hd 64) for gfx950,
// software-pipelined so the matrix pipe and the VALU overlap inside each
// wavefront.
//
// Replaces the backend kernel of GGML_OP_FLASH_ATTN_EXT for the encoder
// calls of voxtral.cpp (src/voxtral.cpp:1580-1613, FA at :1611): the offline
// encoder (hd 64, 20 heads, 1500 frames, bidirectional, mask = null, scale
// 1/sqrt(64)) and the same op under a mask: the realtime encoder's
// sliding-causal window of 750 (src/voxtral.cpp:2179-2190, the mask tensor
// of :1564; 32 heads), as that F16 tensor (MM = 1) or as an implicit mask
// (MM = 2).
//
// Masks. MM = 2, an implicit mask: query row i attends kv j iff
// i + off - W < j <= i + off (W = 0: no lower bound). MM = 1, an F16 mask
// tensor: a pre-pass launch (mask_rows_kernel) records each mask row's live
// interval [lo, hi] when the row is 0 on it and -inf elsewhere, as the
// realtime encoder's window rows are; a workgroup whose rows all have one
// then runs exactly the MM = 2 path with per-row bounds (the same bits as
// the implicit mask). A workgroup with any other row (finite non-zero
// entries, holes) walks every block and adds each score's mask value,
// loaded per element: correct for any mask, and slow. A workgroup's KV
// groups split only the blocks live for some of its 128 rows (at 1500 frames and W = 750 about 28 of the
// 47 blocks), so dead blocks are never copied or computed. A block that is
// not wholly live for all 32 rows of a half gets its dead scores set to
// -inf, in a uniform branch at the top of the half that consumes its S (the
// S block was computed half an iteration earlier, so the MFMAs and softmax
// inside the halves keep their interleaving). A row whose running max is
// still -inf (no live score yet) takes the exact softmax path.
//
// Work decomposition
//   Workgroup = 2 query tiles of 64 rows x 4 KV groups, one wavefront each
//   (8 wavefronts, two per SIMD). KV group g walks its own contiguous share
//   of the 32-position blocks; the groups' partial (O, m, l) are merged
//   through LDS at the end. At 1500 x 20 the grid is 12 x 20 = 240
//   workgroups, one per CU. The workgroups of one head are dealt to one XCD
//   (workgroups go to the 8 XCDs round robin), so that head's K/V stays in
//   one L2. Under a mask each XCD deals its heads' workgroups from the last
//   query tile down (GridMap::make_tiles_desc): the realtime window's 384
//   workgroups run in one and a half rounds, and the first round then holds
//   the long walks (realtime layer, implicit mask, 35.8 -> 27.5 us).
// Why two wavefronts per SIMD: one wavefront issues VALU instructions at
//   about half the SIMD's rate and MFMAs at about 3/4 of the matrix pipe's;
//   two interleaved streams fill both (measured: 1 MFMA + 6 VALU per
//   wavefront runs at 72 cycles per MFMA with two wavefronts, the MFMA pipe
//   75 % busy). Handing the matrix pipe and the VALU to the two wavefronts
//   in turn (one runs all the MFMAs of a block while the other runs its
//   softmax) measured slower (28.2 against 24.9 us per encoder layer): the
//   softmax then runs at one wavefront's VALU rate.
// Why 64 query rows per wavefront: every K and V operand read from LDS feeds
//   two MFMAs (one per 32-row half), half the LDS reads per FLOP of a 32-row
//   wavefront, whose operand reads alone would need the full LDS bandwidth
//   at the MFMA peak.
// Register budget: all of a wavefront's state (O, Q, S, P, K and V operands
//   of both halves, 200-230 VGPRs) stays in registers with no copies, which
//   fits two wavefronts per SIMD (256 VGPRs each).
// Two halves in flight inside the wavefront: the halves A (rows 0-31) and B
//   (rows 32-63) run half an iteration apart. Iteration t (block t of the
//   group):
//     H1: MFMA  O_A += V_t^T P_A(t)^T, S_A(t+1) = K_{t+1} Q_A^T
//         VALU  softmax of S_B(t) -> P_B(t)
//     H2: MFMA  O_B += V_t^T P_B(t)^T, S_B(t+1) = K_{t+1} Q_B^T
//         VALU  softmax of S_A(t+1) -> P_A(t+1)
//   The MFMAs of a half do not depend on that half's VALU work, so the
//   scheduler interleaves them. K_{t+1} is read at the top of iteration t
//   (its block becomes visible at the barrier before) and lands under the
//   PV MFMAs of H1, whose operands are already in registers. V_{t+1} is read
//   in H2 of iteration t, once PV_B(t) has taken V_t's registers as
//   operands.
// K/V staging: a 4-slot LDS ring per KV group; block b sits in slot b % 4
//   and is read (K and V) in iteration b - 1. Block t + 4 is copied into the
//   slot of block t in the middle of iteration t, one barrier after block
//   t's last read (global_load_lds_dwordx4, no staging registers; between
//   the halves, so the copy instructions queue at the texture unit while the
//   MFMAs of H1 run rather than all 8 wavefronts' at once after a barrier);
//   block 4 goes in at the top of iteration 1 (block 0 is read after the
//   prologue's barrier). A block has 2.5 iterations to arrive: at the end of
//   iteration t each wavefront waits only for its own loads of block t + 2
//   (s_waitcnt vmcnt counting the younger blocks still in flight), then one
//   barrier.
// Q is loaded coalesced by the whole workgroup, rounded to f16 and staged in
//   LDS; the output goes out through LDS as full 256-byte rows.
// LDS rows and swizzles, MFMA operand layouts and the row-to-KV permutation
//   are those of fa_prefill.hip (measured conflict-free K and V^T reads).
// Softmax in fp32 with exp2: x = c s - m is one FMA per score, the literal
//   form v_fmamk_f32 when the scale is 1/8 (it issues at twice the rate of
//   the three-register form). Inside the loop P is computed against the
//   running max without reducing the block's max; the sum of P tells when a
//   score passed that max by more than 2^8, and only then is the max raised
//   (O and l rescaled) and P recomputed.
#include "fa_common.h"

#include <type_traits>

namespace vxfa {

namespace pp {
constexpr int D = 64;
constexpr int KS = D / 16;          // S-MFMA k-steps
constexpr int DB = D / 32;          // O^T row blocks
constexpr int BK = 32;              // KV positions per block
constexpr int ROW = D * 2;          // bytes per K/V row
constexpr int BLK = BK * ROW;       // bytes of one matrix block (4 KiB)
constexpr int GRP = 2 * BLK;        // K then V of one group in a ring slot
constexpr float TAU = 8.0f;

// Workgroup shape: NQT query tiles of 64 rows x KVG KV groups (one wavefront
// each), an NS-slot LDS ring per group.
constexpr int NQT = 2;
constexpr int KVG = 4;
constexpr int NS = 4;
constexpr int NW = NQT * KVG;        // wavefronts
constexpr int NT = 64 * NW;
constexpr int BM = 64 * NQT;         // query rows per workgroup
constexpr int SLOT = KVG * GRP;
constexpr int RING = NS * SLOT;
constexpr int QST = BM * ROW;        // Q staging: BM rows of 64 f16
constexpr int NLD = 4 / NQT;         // K (and V) load instructions per wavefront per block
constexpr int PUB = 2 * 32 + 4;      // floats each wavefront publishes per lane for the merge
constexpr int XS = KVG * NQT * PUB * 64 * 4;   // merge area (then the output staging tile)
}  // namespace pp

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14, expcnt 7 and lgkmcnt
// 15 mean "do not wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// every LDS read of this wavefront has returned (s_waitcnt lgkmcnt(0))
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// the main loop's wait: at most k blocks' loads in flight, 0 <= k <= 2
template <int NLD>
__device__ __forceinline__ void wait_blocks_loop(int k) {
    constexpr int L = 2 * NLD;
    if (k >= 2) wait_vmcnt<2 * L>();
    else if (k == 1) wait_vmcnt<L>();
    else wait_vmcnt<0>();
}

// wait until at most k blocks' loads (2 NLD instructions each) are in flight
template <int NLD>
__device__ __forceinline__ void wait_blocks(int k) {
    constexpr int L = 2 * NLD;
    switch (k) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<L>(); break;
        case 2: wait_vmcnt<2 * L>(); break;
        case 3: wait_vmcnt<3 * L>(); break;
        case 4: wait_vmcnt<4 * L>(); break;
        case 5: wait_vmcnt<5 * L>(); break;
        case 6: wait_vmcnt<6 * L>(); break;
        case 7: wait_vmcnt<7 * L>(); break;
        default: wait_vmcnt<8 * L>(); break;
    }
}

// min / max over the 64 lanes (every lane gets the result)
__device__ __forceinline__ int wave_min_i(int x) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) x = min(x, __shfl_xor(x, m, 64));
    return x;
}
__device__ __forceinline__ int wave_max_i(int x) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) x = max(x, __shfl_xor(x, m, 64));
    return x;
}

// min / max / sum over the 16 lanes of a DPP row (every lane of the row gets
// the result; row rotates are VALU operand modifiers, no LDS traffic)
__device__ __forceinline__ int row16_min_i(int x) {
    x = min(x, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(0, x, 0x122, 0xF, 0xF, false));
    return min(x, __builtin_amdgcn_update_dpp(0, x, 0x121, 0xF, 0xF, false));
}
__device__ __forceinline__ int row16_max_i(int x) {
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x122, 0xF, 0xF, false));
    return max(x, __builtin_amdgcn_update_dpp(0, x, 0x121, 0xF, 0xF, false));
}
__device__ __forceinline__ int row16_sum_i(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x122, 0xF, 0xF, false);
    return x + __builtin_amdgcn_update_dpp(0, x, 0x121, 0xF, 0xF, false);
}

// min / max / sum over the 64 lanes: DPP row reductions, then the four rows'
// results read into scalar registers (uniform result, no LDS traffic)
__device__ __forceinline__ int wave_min_dpp(int x) {
    x = row16_min_i(x);
    return min(min(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
               min(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}
__device__ __forceinline__ int wave_max_dpp(int x) {
    x = row16_max_i(x);
    return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
               max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}
__device__ __forceinline__ int wave_sum_dpp(int x) {
    x = row16_sum_i(x);
    return (__builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16)) +
           (__builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48));
}

// The pre-pass of a mask tensor: one wavefront per mask row
// w = (batch bm_i, plane p, row q), w = (bm_i * hm + p) * nq + q, four rows
// per 256-thread block (mask_rows_kernel, and the first blocks of the launch
// that also stages F32 K/V, prep_kernel); writes out[w] = {lo, hi} when the
// row's entries are 0 (+0 or -0) on [lo, hi] and -inf elsewhere, {n, -1}
// when every entry is -inf, {-2, -2} otherwise. The row is read as the
// 16-byte-aligned chunks that cover it (any row alignment; a chunk holds at
// least one byte of the row, so it lies in the same granule as mask data):
// in rounds of 192 chunks, lane s loading chunks c0 + 64 u + s (u < 3, all
// in flight; a chunk past the row's last reloads the last and counts
// nothing). Branch-free per chunk: bit e of `live` is set when entry e lies
// in the row and is not -inf, of `nz` when it is also non-zero; one pass
// gives the first and last live column, their count and whether one is
// non-zero (the row is an interval iff the count is hi - lo + 1), reduced
// over the wavefront. A whole wavefront per row, not a 16-lane DPP row: the
// pre-pass is bound by its VALU work per lane, which a single wavefront per
// SIMD issues at about half the SIMD's rate (1500 realtime-encoder rows:
// 4.8 us with 16 lanes and 12 chunks per lane).
constexpr int kMaskRowChunks = 3;    // chunks per lane per round
constexpr int kMaskRowRound = 64 * kMaskRowChunks;
struct MaskRowArgs {
    const uint16_t* mask;
    int64_t nb1, nb2, nb3;
    int n, nq, hm, nrows;
    int2* out;
};
// Mask row w (w < nrows, uniform over the wavefront) by lane s (0..63);
// every lane calls it (waves past the last row pass w = nrows - 1 and store
// nothing).
__device__ __forceinline__ void mask_row_interval(const MaskRowArgs& m, int w, int s, bool store) {
    const int q = w % m.nq, pb = w / m.nq, p = pb % m.hm, bb = pb / m.hm;
    const char* rowp = (const char*)m.mask + (int64_t)q * m.nb1 + (int64_t)p * m.nb2 + (int64_t)bb * m.nb3;
    const int mis = (int)(reinterpret_cast<uintptr_t>(rowp) & 15);   // even: the mask is 2-byte aligned
    const char* base = rowp - mis;
    const int n = m.n;
    const int nch = (mis + 2 * n + 15) / 16;
    const int nchmax = (14 + 2 * n + 15) / 16;                         // the same loop for every row
    int lo = 0x7fffffff, hi = -1, cnt = 0;
    uint32_t nzall = 0;
    for (int c0 = 0; c0 < nchmax; c0 += kMaskRowRound) {
        u32x4 wv[kMaskRowChunks];
#pragma unroll
        for (int u = 0; u < kMaskRowChunks; ++u) wv[u] = *(const u32x4*)(base + 16 * min(c0 + 64 * u + s, nch - 1));
#pragma unroll
        for (int u = 0; u < kMaskRowChunks; ++u) {
            const int col0 = 8 * (c0 + 64 * u + s) - mis / 2;      // column of the chunk's first entry
            const int elo = max(-col0, 0), ehi = min(n - col0, 8);  // entries [elo, ehi) lie in the row
            const uint32_t valid = ehi > elo ? ((1u << ehi) - 1u) & ~((1u << elo) - 1u) : 0u;
            uint32_t live = 0, nz = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t v = (wv[u][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                const uint32_t l = v != kF16NegInf ? 1u : 0u;
                live |= l << e;
                nz |= (l & ((v & 0x7FFFu) != 0 ? 1u : 0u)) << e;
            }
            live &= valid;
            nzall |= nz & valid;
            const int first = col0 + (int)__builtin_ctz(live | 0x100u);
            const int last = col0 + 31 - (int)__builtin_clz(live | 1u);
            lo = live ? min(lo, first) : lo;
            hi = live ? max(hi, last) : hi;
            cnt += __builtin_popcount(live);
        }
    }
    lo = wave_min_dpp(lo);
    hi = wave_max_dpp(hi);
    cnt = wave_sum_dpp(cnt);
    const int nonzero = wave_max_dpp(nzall != 0 ? 1 : 0);
    if (s == 0 && store)
        m.out[w] = hi < lo ? int2{n, -1} : ((nonzero || cnt != hi - lo + 1) ? int2{-2, -2} : int2{lo, hi});
}

// mask rows [4 bx, 4 bx + 4), one per wavefront
__device__ __forceinline__ void mask_rows_block(const MaskRowArgs& m, uint32_t bx, int tid) {
    const int w = (int)bx * 4 + __builtin_amdgcn_readfirstlane(tid >> 6);
    mask_row_interval(m, min(w, m.nrows - 1), tid & 63, w < m.nrows);
}

__global__ __launch_bounds__(256) void mask_rows_kernel(MaskRowArgs m) {
    mask_rows_block(m, blockIdx.x, (int)threadIdx.x);
}

// The mask pre-pass and F32 K/V staging in one launch of 256-thread blocks:
// blocks [0, nmb) find the intervals of four mask rows each (first, so that
// their memory round trip and VALU work overlap the staging stream), blocks
// [nmb, nmb + 2 sb) stage K (the first sb) and V.
template <bool NT>
__global__ __launch_bounds__(256) void prep_kernel(StageArgs sa, uint32_t sb, uint32_t nmb, MaskRowArgs m) {
    const uint32_t bx = blockIdx.x;
    if (bx < nmb) {
        mask_rows_block(m, bx, (int)threadIdx.x);
        return;
    }
    const uint32_t sx = bx - nmb;
    stage_groups<NT>(sa, sx % sb, (int)(sx / sb), threadIdx.x);
}

template <bool QF16, bool C8, int MM>
__global__ __launch_bounds__(pp::NT) void fa_prefill64_pp(AttnArgs a, GridMap gm, int nblk, int ni) {
    static_assert(MM == 0 || MM == 1 || MM == 2, "no mask, a mask tensor, or an implicit causal / window mask");
    using namespace pp;
    static_assert(NLD * NQT == 4, "a block's 4 load instructions per matrix split evenly");
    static_assert(8 * 2 * NLD < 64 && NS <= 8, "vmcnt range of wait_blocks");
    static_assert(XS <= RING + QST && BM * 256 <= RING + QST, "merge and output staging fit the LDS");
    __shared__ __attribute__((aligned(16))) char smem[RING + QST];

    // ---- XCD-aware position of this workgroup --------------------------------
    int qg, h, b, hk, bkv;
    gm.locate(blockIdx.x, qg, h, b, hk, bkv);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / NQT;
    const int wq = wave % NQT;
    const int nl = lane & 31;
    const int hh = lane >> 5;
    const int qw0 = qg * BM;                  // first query row of the workgroup
    const float c = fabsf(a.scale_log2);      // |scale| * log2(e); a negative scale is folded into Q
    const char* kb = (const char*)a.k + (int64_t)hk * a.k_nb2 + (int64_t)bkv * a.k_nb3;
    const char* vb = (const char*)a.v + (int64_t)hk * a.v_nb2 + (int64_t)bkv * a.v_nb3;

    // MM = 1: the intervals of the workgroup's 128 rows, rows l and 64 + l on
    // lane l (loaded before Q, so that their wait leaves the Q loads in
    // flight; rows past n_q load row n_q - 1 and count as empty). Loads here
    // are unconditional: a load under a branch makes the compiler wait for
    // it at the join, before the K/V copies are issued.
    int2 iv[2] = {int2{0, 0}, int2{0, 0}};
    if constexpr (MM == 1) {
        const int2* tab = a.mask_rows + ((int64_t)(b % a.bm) * a.hm + (h % a.hm)) * a.nq;
#pragma unroll
        for (int u = 0; u < 2; ++u) iv[u] = tab[min(qw0 + 64 * u + lane, a.nq - 1)];
    }

    // ---- Q: coalesced loads by the whole workgroup (issued first, so their
    // latency overlaps the first K/V blocks) -----------------------------------
    // Staged in LDS as f16 rows of 128 bytes, 16-byte chunk j of row r at
    // position j ^ (r & 7). F32 Q: thread i takes 16-byte chunks i + NT u of
    // the BM x 16 chunks; F16 Q: of the BM x 8 chunks.
    // Q is read once and O written once (whole 256-byte rows): nontemporal
    // loads and stores (21.7 -> 20.3 us per layer measured on one box).
    // Rows past n_q load row n_q - 1 (unconditional loads, see above) and
    // are staged as zeros.
    constexpr int QCH = QF16 ? 8 : 16;         // 16-byte global chunks per row
    constexpr int QPT = BM * QCH / NT;         // per thread
    floatx4 qraw[QPT];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int i = tid + NT * u;
        const int r = i / QCH, cch = i % QCH;
        const int row = min(qw0 + r, a.nq - 1);
        qraw[u] = __builtin_nontemporal_load((const floatx4*)((const char*)a.q + (int64_t)row * a.q_nb1 +
                                                              (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3 + cch * 16));
    }

    // MM = 1: whether every row of the workgroup has a live interval (mslow
    // = false), the union of the intervals (uniform: scalar registers, so
    // the loop bounds stay scalar; every wavefront reduces all 128 rows, no
    // barrier), and the intervals of the lane's rows in the two halves
    // (rows 64 wq + 32 x + l % 32)
    bool mslow = false;
    int wlo = 0x7fffffff, whi = -1;
    int2 ivl[2] = {int2{0, 0}, int2{0, 0}};
    if constexpr (MM == 1) {
        bool non = false;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (qw0 + 64 * u + lane >= a.nq) iv[u] = int2{a.nkv, -1};
            non = non || iv[u].x == -2;
            if (iv[u].x >= 0 && iv[u].x <= iv[u].y) {
                wlo = min(wlo, iv[u].x);
                whi = max(whi, iv[u].y);
            }
        }
        wlo = __builtin_amdgcn_readfirstlane(wave_min_i(wlo));
        whi = __builtin_amdgcn_readfirstlane(wave_max_i(whi));
        mslow = __any(non);
        static_assert(NQT == 2, "a wavefront's 64 rows are iv[wq] of the workgroup's 128");
        const int2 mine = wq ? iv[1] : iv[0];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            ivl[x].x = __shfl(mine.x, 32 * x + nl, 64);
            ivl[x].y = __shfl(mine.y, 32 * x + nl, 64);
        }
    }
    // blocks [blo, blo + nblk) hold the live KV positions of the workgroup's
    // rows (all of them without a mask, or with mslow);
    // KV group kg takes [bs, bs + ng)
    int blo = 0;
    if constexpr (MM == 1) {
        if (!mslow) {
            if (whi < wlo) {
                nblk = 0;
            } else {
                blo = wlo / BK;
                nblk = (whi + BK) / BK - blo;
            }
            ni = (nblk + KVG - 1) / KVG;
        }
    }
    if constexpr (MM == 2) {
        const int64_t q1 = min(qw0 + BM, a.nq) - 1;      // the workgroup's last real row
        int64_t lo = a.im_window > 0 ? (int64_t)qw0 + a.im_offset - a.im_window + 1 : 0;
        int64_t hi = q1 + a.im_offset + 1;                // exclusive
        lo = lo < 0 ? 0 : lo;
        hi = hi > a.nkv ? a.nkv : hi;
        if (hi <= lo) lo = hi = 0;
        blo = (int)(lo / BK);
        nblk = (int)((hi + BK - 1) / BK) - blo;
        ni = (nblk + KVG - 1) / KVG;
    }
    // The rest of the kernel, in two copies under a mask tensor (MM = 1):
    // workgroups whose rows are all intervals, and workgroups that add the
    // mask per element (SLOW). With the per-element code inside the one
    // pipelined loop the compiler lays out the interval path differently
    // (fewer unrolled MFMA groups, twice the register moves), measured at
    // 3.7 us more per realtime-encoder layer.
    auto rest = [&](auto slow_tag) __attribute__((always_inline)) {
        constexpr bool SLOW = decltype(slow_tag)::value;
        static_assert(!SLOW || MM == 1, "the per-element path is the mask tensor's");
        const int bs = blo + min(kg * ni, nblk);
        const int ng = min(ni, blo + nblk - bs);


        // ---- block loads: global -> LDS ring -------------------------------------
        // Instruction i of wavefront wq fills rows [8 (NQT i + wq), + 8) of the
        // group's block; lane l writes LDS chunk l % 8 of row + l / 8, which holds
        // the row's chunk (l % 8) ^ swizzle(row). A block's rows start at a
        // scalar base plus a 32-bit lane offset (row strides are below 8 MiB,
        // checked by the host); the partial last block clamps rows past n_kv to
        // row n_kv - 1.
        uint32_t ldk[NLD], ldv[NLD];
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int r = 8 * (NQT * i + wq) + (lane >> 3);
            ldk[i] = (uint32_t)r * (uint32_t)a.k_nb1 + ((lane & 7) ^ swz_k<D>(r)) * 16;
            ldv[i] = (uint32_t)r * (uint32_t)a.v_nb1 + ((lane & 7) ^ swz_v<D>(r)) * 16;
        }
        const uint32_t lds0 = lds_offset(smem) + kg * GRP;
        auto issue = [&](int blk) {   // blk: index within the group, < ng
            const int kv0 = (bs + blk) * BK;
            const uint32_t kd = lds0 + (blk % NS) * SLOT, vd = kd + BLK;
            const char* kst = kb + (int64_t)kv0 * a.k_nb1;
            const char* vst = vb + (int64_t)kv0 * a.v_nb1;
            if (kv0 + BK <= a.nkv) {
#pragma unroll
                for (int i = 0; i < NLD; ++i) {
                    const uint32_t r0b = 8 * (NQT * i + wq) * ROW;
                    dma16(kst, ldk[i], kd + r0b);
                    dma16(vst, ldv[i], vd + r0b);
                }
            } else {
                // once per head: the offsets are recomputed here rather than held
                // in registers across the loop (the empty asm keeps them here)
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const int rmax = a.nkv - 1 - kv0;   // last valid row of the block (kv0 < n_kv)
#pragma unroll
                for (int i = 0; i < NLD; ++i) {
                    const int r0 = 8 * (NQT * i + wq);
                    const int r = r0 + (ln >> 3);
                    const int rc = min(r, rmax);
                    dma16(kst, (uint32_t)rc * (uint32_t)a.k_nb1 + ((ln & 7) ^ swz_k<D>(r)) * 16, kd + r0 * ROW);
                    dma16(vst, (uint32_t)rc * (uint32_t)a.v_nb1 + ((ln & 7) ^ swz_v<D>(r)) * 16, vd + r0 * ROW);
                }
            }
        };
        const int npre = min(ng, NS - 1);
        for (int blk = 0; blk < npre; ++blk) issue(blk);

        // ---- Q: wait for its loads only, round to f16 (ggml's Q conversion, sign
        // of the scale folded in), stage in LDS ------------------------------------
        // (the npre blocks' loads were issued after the Q loads and may remain)
        wait_blocks<NLD>(npre);
        {
            char* qs = smem + RING;
            const float sg = a.scale_log2 < 0.f ? -1.0f : 1.0f;
#pragma unroll
            for (int u = 0; u < QPT; ++u) {
                const int i = tid + NT * u;
                const int r = i / QCH, cch = i % QCH;
                const floatx4 qv = qw0 + r < a.nq ? qraw[u] : floatx4{0.f, 0.f, 0.f, 0.f};
                if (QF16) {
                    const half8 v = __builtin_bit_cast(half8, qv) * (_Float16)sg;
                    *(half8*)(qs + r * ROW + ((cch ^ (r & 7)) * 16)) = v;
                } else {
                    half4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = (_Float16)(qv[e] * sg);
                    *(half4*)(qs + r * ROW + (((cch >> 1) ^ (r & 7)) * 16) + (cch & 1) * 8) = v;
                }
            }
        }

        // ---- operand reads from LDS (offsets within a group's block) ----------------
        // K: A-operand row nl of the 32-block is K row krow (the row-to-KV
        // permutation), chunk 2 ks + hh.
        int kaddr[KS];
        {
            const int am = nl >> 3, ahb = (nl >> 2) & 1, ab = nl & 3;
            const int krow = ahb ? 16 + ((am + 2) & 3) * 4 + ab : 4 * am + ab;
            const int kx = hh ^ swz_k<D>(krow);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kaddr[ks] = krow * ROW + ((2 * ks) ^ kx) * 16;
        }
        // V^T: operand (cc, db) covers the 8 positions of P operand cc, read as two
        // transposed 8-byte loads 4 rows apart.
        int vaddr[2][DB];
        {
            const int vq = (lane & 15) >> 2;
            const int clo = 2 * ((lane & 31) >> 4) + ((lane & 3) >> 1);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    vaddr[cc][db] = ((hh ? 24 - 8 * cc : 8 * cc) + vq) * ROW + ((4 * db + clo) ^ swz_v<D>(vq)) * 16 +
                                    (lane & 1) * 8;
        }
        auto read_k = [&](int blk, half8 (&kr)[KS]) {
            const char* base = smem + (blk % NS) * SLOT + kg * GRP;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kr[ks] = *(const half8*)(base + kaddr[ks]);
        };
        auto read_v = [&](int blk, half8 (&vr)[2][DB]) {
            const char* base = smem + (blk % NS) * SLOT + kg * GRP + BLK;
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const half4 lo4 = lds_read_tr16(base + vaddr[cc][db]);
                    const half4 hi4 = lds_read_tr16(base + vaddr[cc][db] + 4 * ROW);
                    vr[cc][db] = half8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                }
        };

        // ---- MFMA groups and the softmax -------------------------------------------
        auto s_mfma = [&](floatx16& s, const half8 (&q)[KS], const half8 (&kr)[KS]) {
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[0], q[0], floatx16{}, 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < KS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[ks], q[ks], s, 0, 0, 0);
        };
        auto pv_mfma = [&](floatx16 (&o)[DB], const half8 (&p)[2], const half8 (&vr)[2][DB]) {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < DB; ++db) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[cc][db], p[cc], o[db], 0, 0, 0);
        };
        // positions of the partial block blk at or past n_kv score -inf
        auto tail_fix = [&](floatx16& sc, int blk) {
            const int kv0 = (bs + blk) * BK;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (kv0 + pf_kv_of(hh, j) >= a.nkv) sc[j] = -INFINITY;
        };
        // MM = 1 / 2: the live positions [rlo, rhi] of the lane's row in each
        // half (clamped to [-1, n_kv]), and per half the largest lower bound and
        // the smallest upper bound over its 32 rows (a block inside both is
        // wholly live for the half)
        int rlo[2] = {0, 0}, rhi[2] = {0, 0}, hlo[2] = {0, 0}, hhi[2] = {0, 0};
        if constexpr (MM == 1) {
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                rlo[x] = ivl[x].x;
                rhi[x] = ivl[x].y;
                // (lanes l and l + 32 hold the same row; uniform results)
                hlo[x] = __builtin_amdgcn_readfirstlane(wave_max_i(rlo[x]));
                hhi[x] = __builtin_amdgcn_readfirstlane(wave_min_i(rhi[x]));
            }
        }
        if constexpr (MM == 2) {
            auto clampkv = [&](int64_t x) { return (int)(x < -1 ? -1 : (x > a.nkv ? a.nkv : x)); };
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                const int64_t r0 = (int64_t)qw0 + 64 * wq + 32 * x;
                const int64_t wb = a.im_window > 0 ? a.im_offset - a.im_window + 1 : INT64_MIN / 2;
                rlo[x] = clampkv(r0 + nl + wb);
                rhi[x] = clampkv(r0 + nl + a.im_offset);
                hlo[x] = clampkv(r0 + 31 + wb);
                hhi[x] = clampkv(r0 + a.im_offset);
            }
        }
        // MM = 1 / 2: block blk (of this group) for half x; a uniform branch,
        // taken only for blocks not wholly live for the half's rows. SLOW:
        // every score gets its mask value (per element loads; -inf, and
        // a position past n_kv, remove it; a finite value m adds m / |scale|,
        // so that c s becomes c s + m log2(e)). The lane's mask row (rows past
        // n_q read row n_q - 1; their outputs are not stored) is addressed here
        // rather than held in registers across the loop (the empty asm keeps
        // the computation here).
        auto mask_fix = [&](floatx16& sc, int blk, int x) {
            if constexpr (SLOW) {
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const int row = min(qw0 + 64 * wq + 32 * x + (ln & 31), a.nq - 1);
                const uint16_t* mr = (const uint16_t*)((const char*)a.mask + (int64_t)(h % a.hm) * a.m_nb2 +
                                                       (int64_t)(b % a.bm) * a.m_nb3 + (int64_t)row * a.m_nb1);
                const int kv0 = (bs + blk) * BK;
                const float inv_sc = kLog2e / c;
                uint16_t mv[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) mv[j] = mr[min(kv0 + pf_kv_of(ln >> 5, j), a.nkv - 1)];
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    sc[j] = (mv[j] == kF16NegInf || kv0 + pf_kv_of(ln >> 5, j) >= a.nkv)
                                ? -INFINITY
                                : fmaf(f16_bits_to_f32(mv[j]), inv_sc, sc[j]);
            } else if constexpr (MM != 0) {
                const int kv0 = (bs + blk) * BK;
                if (!(kv0 >= hlo[x] && kv0 + BK - 1 <= hhi[x])) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int kv = kv0 + pf_kv_of(hh, j);
                        sc[j] = (kv < rlo[x] || kv > rhi[x]) ? -INFINITY : sc[j];
                    }
                }
            }
        };
        // P = 2^(c s - m) for the lane's 16 scores, as two f16 B operands, and
        // their sum. With C8 (scale exactly 1/8) c is a literal and x = c s - m
        // compiles to v_fmamk_f32, which issues at twice the rate of the
        // three-register v_fma_f32; -m has to reach it as a plain register (a
        // negation folded into the FMA would force the three-register form), so
        // it passes through an empty asm. (Every instruction that reads an MFMA
        // result must be one the compiler sees: it alone inserts the wait states
        // such a read needs.)
        const half2 ones = {(_Float16)1.0f, (_Float16)1.0f};
        auto exps = [&](const floatx16& sc, float m, half8 (&p)[2]) -> float {
            float nm = (m == -INFINITY) ? 0.f : -m;
            asm("" : "+v"(nm));
            float ls[2] = {0.f, 0.f};
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    p[cc][i] = (_Float16)exp2_fast(fmaf(sc[8 * cc + i], C8 ? 0.18033688f : c, nm));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const half2 p2 = {p[cc][2 * i], p[cc][2 * i + 1]};
                    ls[i & 1] = __builtin_amdgcn_fdot2(p2, ones, ls[i & 1], false);
                }
            }
            return ls[0] + ls[1];
        };
        // the block's max (log2 units) over the lane pair
        auto block_max = [&](const floatx16& sc) -> float {
            float r = sc[0];
#pragma unroll
            for (int j = 1; j < 16; ++j) r = fmaxf(r, sc[j]);
            return pair32_max(r) * c;
        };
        // raise the running max to mx: rescale O and l
        auto raise = [&](float mx, float& m, float& l, floatx16 (&o)[DB]) {
            const float mnew = fmaxf(m, mx);
            const float ms = (mnew == -INFINITY) ? 0.f : mnew;
            const float alpha = exp2_fast(m - ms);
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 16; ++j) o[db][j] *= alpha;
            l *= alpha;
            m = mnew;
        };
        // With a mask, rows past n_q (their outputs are not stored) take no part
        // in the wavefront's choice of the exact path: its rows then see the same
        // choices under any two masks that agree on the real rows (an implicit
        // mask and the same mask as a tensor give the same bits). Such a row may
        // keep m = -inf and turn its own P, l and O to inf / NaN; each row's
        // values stay in its own column of P and O and are dropped at the store.
        const bool real_a = MM == 0 || qw0 + 64 * wq + nl < a.nq;
        const bool real_b = MM == 0 || qw0 + 64 * wq + 32 + nl < a.nq;
        // softmax of one block, max first (blocks outside the pipelined loop)
        auto softmax_exact = [&](const floatx16& sc, float& m, float& l, floatx16 (&o)[DB], half8 (&p)[2], bool real) {
            const float mx = block_max(sc);
            if (__any(mx > m + TAU && real)) raise(mx, m, l, o);
            l += exps(sc, m, p);
        };
        // Softmax inside the pipelined loop. P is computed against the current
        // running max m with no block max at all: a score more than TAU above m
        // makes some P > 2^TAU, so the lane's sum of its 16 P exceeds 2^TAU (and is
        // inf or NaN past the f16 range). Only then (rare once m has settled) is
        // the block max reduced, O and l rescaled and P recomputed; a large sum of
        // moderate P can also take that path, which is harmless. Once m is raised
        // every P of later blocks stays below 2^TAU unless a new larger score
        // arrives, which the same test catches.
        // The basic block of each half (closed by that branch) holds its 8 MFMAs
        // and the softmax's fast path, which the compiler's max-ILP scheduler
        // interleaves (the file is built with it). Under the default scheduler
        // the kernel pinned the order with scheduling groups (in H1 the 4 K
        // operand reads, then 12 VALU instructions, then one MFMA per 5 VALU;
        // in H2 one MFMA per 6); with max-ILP those groups measured slower
        // (encoder layer 21.05 against 20.61 us, realtime encoder implicit
        // 27.35 against 26.94, alternating A/B on one box).
        auto softmax_spec = [&](const floatx16& sc, float& m, float& l, floatx16 (&o)[DB], half8 (&p)[2],
                                bool real) {
            float ls = exps(sc, m, p);
            // 2^TAU (also true for inf / NaN); with a mask, also a row that has
            // no live score yet (its P above were taken against m = 0)
            bool slow = !(ls <= 256.0f);
            if constexpr (MM != 0) slow = (slow || m == -INFINITY) && real;
            if (__any(slow)) {
                raise(block_max(sc), m, l, o);
                ls = exps(sc, m, p);
            }
            l += ls;
        };

        floatx16 oa[DB], ob[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db) { oa[db] = floatx16{}; ob[db] = floatx16{}; }
        float ma = -INFINITY, mb = -INFINITY, la = 0.f, lb = 0.f;
        floatx16 sa, sb;
        half8 pa[2], pb[2];
        half8 kr[KS];
        half8 vr[2][DB];

        // Full blocks of this group run through the pipelined loop; the partial
        // last block of the KV range (only the last group can hold it) is computed
        // on its own after them, so the loop body needs no position checks.
        const bool part = ng > 0 && (bs + ng) * BK > a.nkv;
        const int nf = ng - (part ? 1 : 0);

        // ---- prologue: blocks 0 and 1 landed; Q operands; S_A(0), S_B(0), P_A(0) ----
        wait_blocks<NLD>(max(npre - 2, 0));
        __syncthreads();   // Q staged, blocks 0 and 1 visible
        half8 qa[KS], qb[KS];
        {
            const char* qs = smem + RING;
            const int ra = 64 * wq + nl, rb = ra + 32;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                qa[ks] = *(const half8*)(qs + ra * ROW + (((2 * ks + hh) ^ (ra & 7)) * 16));
                qb[ks] = *(const half8*)(qs + rb * ROW + (((2 * ks + hh) ^ (rb & 7)) * 16));
            }
        }
        if (nf > 0) {
            read_k(0, kr);
            read_v(0, vr);
            s_mfma(sa, qa, kr);
            s_mfma(sb, qb, kr);
            mask_fix(sa, 0, 0);
            mask_fix(sb, 0, 1);
            softmax_exact(sa, ma, la, oa, pa, real_a);
            // the loop's softmax needs a finite running max to start from
            mb = block_max(sb);
        }

        // ---- main loop: full blocks 0 .. nf - 2 ------------------------------------
        // Copies: blocks 0 .. NS - 2 before the loop; between the halves of
        // iteration 0 block NS - 1 (its slot is still unused), of iteration
        // t >= 1 block t + NS into the slot of block t (read in iteration t - 1,
        // before its barrier); block NS at the top of iteration 1 (block 0 is
        // read after the prologue's barrier). At the end of iteration t block
        // t + 2 must have landed (read at the top of iteration t + 1). Every
        // wavefront passes one barrier per block of the longest group (ni), plus
        // the prologue's and the merge's.
        for (int t = 0; t + 1 < nf; ++t) {
            if (t == 1 && NS < ng) issue(NS);
            read_k(t + 1, kr);
            if (t > 0) mask_fix(sb, t, 1);   // S_B(t), from H2 of the previous iteration
            // H1: PV_A(t), S_A(t+1) on the matrix pipe; softmax of S_B(t). The
            // MFMAs come first in the source so they share a basic block with
            // the softmax's fast path (its rare rescale branch closes the block)
            // and the scheduler can interleave the two; PV_A first, as its
            // operands are in registers while K_{t+1} lands.
            pv_mfma(oa, pa, vr);
            s_mfma(sa, qa, kr);
            softmax_spec(sb, mb, lb, ob, pb, real_b);
            if ((t == 0 ? NS - 1 : t + NS) < ng) issue(t == 0 ? NS - 1 : t + NS);
            // H2: PV_B(t), S_B(t+1); softmax of S_A(t+1)
            mask_fix(sa, t + 1, 0);
            pv_mfma(ob, pb, vr);
            read_v(t + 1, vr);   // V_{t+1}: its block is visible since the previous barrier
            s_mfma(sb, qb, kr);
            softmax_spec(sa, ma, la, oa, pa, real_a);
            // blocks issued so far: up to NS - 1 (t = 0), t + NS (t >= 1)
            const int last = min(t >= 1 ? t + NS : NS - 1, ng - 1);
            wait_blocks_loop<NLD>(last - (t + 2));   // 2 at most: last <= t + NS
            __syncthreads();
        }
        // (no loads are issued from here on)
        if (nf > 0) {
            // last full block: PV_A, softmax of S_B, PV_B
            if (nf > 1) mask_fix(sb, nf - 1, 1);
            pv_mfma(oa, pa, vr);
            softmax_exact(sb, mb, lb, ob, pb, real_b);
            pv_mfma(ob, pb, vr);
            wait_vmcnt<0>();
            __syncthreads();
        }
        if (part) {
            // the partial block, unpipelined
            const int tp = nf;
            read_k(tp, kr);
            s_mfma(sa, qa, kr);
            s_mfma(sb, qb, kr);
            read_v(tp, vr);
            tail_fix(sa, tp);
            tail_fix(sb, tp);
            mask_fix(sa, tp, 0);
            mask_fix(sb, tp, 1);
            softmax_exact(sa, ma, la, oa, pa, real_a);
            softmax_exact(sb, mb, lb, ob, pb, real_b);
            pv_mfma(oa, pa, vr);
            pv_mfma(ob, pb, vr);
            __syncthreads();
        }
        for (int tt = ng; tt < ni; ++tt) __syncthreads();

        // ---- merge the KV groups through LDS (the ring is free), normalise ------------
        // Every wavefront publishes its (O, m, l) as 17 chunks of 4 floats per lane,
        // chunk-major (chunk c of lane l at floats 256 c + 4 l: one 16-byte write
        // and read per chunk, the 64 lanes' chunks contiguous): chunk c < 16 holds
        // O elements 4c .. 4c + 3 (element e = 32 x + 16 v + j is accumulator j of
        // vector v of half x), chunk 16 holds (m_A, m_B, l_A, l_B). Wavefront
        // (kg, wq) then merges elements [16 kg, 16 kg + 16) of query tile wq over
        // all groups (one O vector of one half), in group order, and after a
        // barrier (the staging tile overlaps the published data) writes them
        // normalised to the staging tile, row r at r * 256 bytes with 16-byte
        // chunk j at position j ^ (r & 15); then all wavefronts store full rows.
        constexpr int EPW = 64 / KVG;                   // elements merged per wavefront
        static_assert(EPW % 4 == 0 && EPW <= 32, "a wavefront's elements lie in one half");
        static_assert(PUB == 17 * 4, "published chunks");
        float* xs = (float*)smem;
        char* ost = smem;
        {
            floatx4* w = (floatx4*)(xs + (kg * NQT + wq) * PUB * 64) + lane;
#pragma unroll
            for (int ci = 0; ci < 16; ++ci) {
                const floatx16& o = (ci < 8) ? oa[(ci % 8) / 4] : ob[(ci % 8) / 4];
                const int j0 = 4 * (ci % 4);
                w[ci * 64] = floatx4{o[j0], o[j0 + 1], o[j0 + 2], o[j0 + 3]};
            }
            w[16 * 64] = floatx4{ma, mb, la, lb};
        }
        __syncthreads();
        const int e0 = kg * EPW;        // first element: 0..31 half A, 32..63 half B
        const int x = e0 / 32;
        floatx4 res[EPW / 4];
        {
            float mg[KVG], lg[KVG];
            float M = -INFINITY;
#pragma unroll
            for (int g = 0; g < KVG; ++g) {
                const floatx4 ml = ((const floatx4*)(xs + (g * NQT + wq) * PUB * 64))[16 * 64 + lane];
                mg[g] = x ? ml[1] : ml[0];
                lg[g] = x ? ml[3] : ml[2];
                M = fmaxf(M, mg[g]);
            }
            const float Ms = (M == -INFINITY) ? 0.f : M;
            float wg[KVG];
            float lsum = 0.f;
#pragma unroll
            for (int g = 0; g < KVG; ++g) {
                wg[g] = exp2_fast(mg[g] - Ms);
                lsum = fmaf(wg[g], lg[g], lsum);
            }
            const float lt = pair32_sum(lsum);
            const float inv = (lt == 0.f) ? 0.f : 1.0f / lt;
#pragma unroll
            for (int g = 0; g < KVG; ++g) wg[g] *= inv;
            floatx4 og[KVG][EPW / 4];
#pragma unroll
            for (int g = 0; g < KVG; ++g)
#pragma unroll
                for (int q = 0; q < EPW / 4; ++q)
                    og[g][q] = ((const floatx4*)(xs + (g * NQT + wq) * PUB * 64))[(e0 / 4 + q) * 64 + lane];
#pragma unroll
            for (int q = 0; q < EPW / 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float acc = 0.f;
#pragma unroll
                    for (int g = 0; g < KVG; ++g) acc = fmaf(wg[g], og[g][q][e], acc);
                    res[q][e] = acc;
                }
        }
        __syncthreads();   // every read of the published data is done
        {
            const int row = 64 * wq + 32 * x + nl;
#pragma unroll
            for (int q = 0; q < EPW / 4; ++q) {
                const int eh = e0 - 32 * x + 4 * q;              // element within the half: 16 db + 4 a4
                const int ch = 8 * (eh / 16) + 2 * ((eh % 16) / 4) + hh;   // dims 4 ch .. 4 ch + 3
                *(floatx4*)(ost + row * 256 + ((ch ^ (row & 15)) * 16)) = res[q];
            }
        }
        __syncthreads();
        // ---- store: dst[b][row][h][0..63], 16 threads per 256-byte row -------------
#pragma unroll
        for (int u = 0; u < BM * 16 / NT; ++u) {
            const int i = tid + NT * u;
            const int r = i >> 4, ch = i & 15;
            const int row = qw0 + r;
            if (row < a.nq) {
                const floatx4 v = *(const floatx4*)(ost + r * 256 + ((ch ^ (r & 15)) * 16));
                __builtin_nontemporal_store(v, (floatx4*)(a.dst + (((int64_t)b * a.nq + row) * a.hq + h) * D + 4 * ch));
            }
        }
    };
    if constexpr (MM == 1) {
        if (mslow) rest(std::true_type{});
        else rest(std::false_type{});
    } else {
        rest(std::false_type{});
    }
}

// hd 64 without a mask or with an implicit causal / window mask: 128 query
// rows x 4 KV groups per workgroup.
template <int MM>
static void launch_pp_mm(const AttnArgs& a, const GridMap& gm, int nblk, int ni, bool is_c8, const dim3& grid,
                         const dim3& block, hipStream_t st) {
    if (a.q_f16) {
        if (is_c8) hipLaunchKernelGGL((fa_prefill64_pp<true, true, MM>), grid, block, 0, st, a, gm, nblk, ni);
        else hipLaunchKernelGGL((fa_prefill64_pp<true, false, MM>), grid, block, 0, st, a, gm, nblk, ni);
    } else {
        if (is_c8) hipLaunchKernelGGL((fa_prefill64_pp<false, true, MM>), grid, block, 0, st, a, gm, nblk, ni);
        else hipLaunchKernelGGL((fa_prefill64_pp<false, false, MM>), grid, block, 0, st, a, gm, nblk, ni);
    }
}

hipError_t launch_mask_prep(const AttnArgs& a, const StageReq* stage, hipStream_t st) {
    if (!a.mask || !a.mask_rows) return hipErrorInvalidValue;
    StageArgs sa;
    uint32_t sb = 0;
    bool snt = false;
    if (stage && !make_stage_args(*stage, sa, sb, snt)) return hipErrorInvalidValue;
    const int64_t nrows = (int64_t)a.nq * a.hm * a.bm;
    if (nrows <= 0 || nrows > 0x7fffffff - 15) return hipErrorInvalidValue;
    const MaskRowArgs m{a.mask, a.m_nb1, a.m_nb2, a.m_nb3, a.nkv, a.nq, a.hm, (int)nrows, a.mask_rows};
    const uint32_t nmb = (uint32_t)((nrows + 3) / 4);   // four rows per block
    if (sb > 0) {
        const uint64_t nb = 2ull * sb + nmb;
        if (nb > 0x7fffffffull) return hipErrorInvalidValue;
        if (snt) hipLaunchKernelGGL(prep_kernel<true>, dim3((unsigned)nb), dim3(256), 0, st, sa, sb, nmb, m);
        else hipLaunchKernelGGL(prep_kernel<false>, dim3((unsigned)nb), dim3(256), 0, st, sa, sb, nmb, m);
    } else {
        hipLaunchKernelGGL(mask_rows_kernel, dim3(nmb), dim3(256), 0, st, m);
    }
    return hipGetLastError();
}

hipError_t launch_prefill64_pp(const AttnArgs& a, const StageReq* stage, hipStream_t st) {
    using namespace pp;
    const int nqg = (a.nq + BM - 1) / BM;
    const int nblk = (a.nkv + BK - 1) / BK;
    const int ni = (nblk + KVG - 1) / KVG;
    const int64_t nwg = (int64_t)nqg * a.hq * a.b;
    if (nwg <= 0 || nwg > 0x7fffffff || nblk <= 0) return hipErrorInvalidValue;
    // |scale| * log2(e) equal, bit for bit, to the literal in the kernel
    const float c8 = 0.125f * kLog2e;
    const bool is_c8 = fabsf(a.scale_log2) == c8 && __builtin_bit_cast(uint32_t, c8) == 0x3e38aa3bu;
    // under a mask, heavy query tiles first (a causal or window mask makes
    // later tiles walk more blocks)
    const GridMap gm = (a.mask || a.im_causal) ? GridMap::make_tiles_desc((int)nwg, nqg, a.hq, a.hkv, a.b, a.bk)
                                               : GridMap::make((int)nwg, nqg, a.hq, a.hkv, a.b, a.bk);
    const dim3 grid((unsigned)nwg), block(NT);
    if (a.mask) {
        const hipError_t e = launch_mask_prep(a, stage, st);
        if (e != hipSuccess) return e;
        launch_pp_mm<1>(a, gm, nblk, ni, is_c8, grid, block, st);
    } else {
        if (stage) {
            const hipError_t e = launch_to_f16_kv(*stage, st);
            if (e != hipSuccess) return e;
        }
        if (a.im_causal) launch_pp_mm<2>(a, gm, nblk, ni, is_c8, grid, block, st);
        else launch_pp_mm<0>(a, gm, nblk, ni, is_c8, grid, block, st);
    }
    return hipGetLastError();
}

}  // namespace vxfa
