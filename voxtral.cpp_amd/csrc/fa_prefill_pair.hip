// fa_prefill_pair.hip — short masked prefill for gfx950: hd 128, n_kv <= 512,
// 32-row query tiles paired from both ends of the sequence.
//
// Replaces the backend kernel of GGML_OP_FLASH_ATTN_EXT for voxtral.cpp's
// decoder prefill: GQA 32/8, hd 128, causal mask (src/voxtral.cpp:1802; mask
// filled by fill_causal_mask :2104-2111 and cast at :1801), or the same call
// with the mask given as a formula (vxfa_flash_attn_ext_implicit).
//
// Why a kernel of its own: at this size the work is a few microseconds of
// matrix time spread over 224 workgroups, and a kernel that walks the KV axis
// in steps pays a memory round trip per step on its longest walk. Here every
// wavefront computes (about) one block, and all of a workgroup's loads are in
// flight at once.
//
// Work decomposition
//   A head's query rows form nt = ceil(n_q / 32) tiles. Workgroup p of a head
//   takes tiles A = p and B = nt - 1 - p (B alone when they meet). Under a
//   causal mask tile i meets floor(i / 2) + 1 live 64-position KV tiles, so
//   every pair holds about the same number of live (tile, KV tile) blocks:
//   8 at n_q = 439, one per wavefront.
//   Block classes: dead (skipped), all-zero mask (computed without the mask)
//   or mixed (mask values added). With an implicit mask they follow from the
//   formula; with a mask tensor each wavefront first reads the mask of two
//   candidate blocks, (B, w) and (A, 7 - w), as whole row segments, and
//   classifies them; with a mask tensor whose rows' live intervals a pre-pass
//   has found (MM 3: the launch that stages F32 K/V runs it) they follow
//   from the intervals, and a tile whose rows are all intervals also forms
//   its mixed blocks' mask words from them.
//   Assignment: B's live blocks go to wavefronts 0 .. wB - 1, A's to the rest
//   in reverse order (wB in proportion to the live counts), so under a causal
//   mask each wavefront computes the block it classified. With at most 8 live KV tiles per query tile
//   no wavefront gets more than two blocks (checked for every pair of live
//   counts on the CPU); it takes one max over both, so O needs no rescale.
//   Merge: every wavefront publishes (O, m, l) to LDS; the wavefronts of a
//   tile then each merge and store a quarter (or so) of its elements.
// Memory, in three phases through one 128 KiB LDS area: every live K tile of
//   the pair is copied in once (direct global-to-LDS copies of whole rows,
//   16 KiB per tile, at most 8) and the wavefronts compute S from it; after a
//   barrier the V tiles are copied over them while the softmax runs; then
//   O^T = V^T P^T. Both tiles' wavefronts share every tile. (K read straight
//   into the operand registers measured slower: each load instruction touches
//   32 B of each of 32 rows.) Q of both tiles is rotated
//   (vxfa_flash_attn_ext_rope: ggml's rope mode 0 at each row's position),
//   rounded to f16 (ggml's Q conversion) and staged in LDS.
// MFMA layouts, the row-to-KV permutation within a 32-position block, the V
//   tile's XOR swizzle and the transposed V^T reads are those of
//   fa_prefill.hip (v_mfma_f32_32x32x16_f16: S^T = K Q^T, O^T = V^T P^T).
#include "fa_common.h"

#include <type_traits>

namespace vxfa {

namespace pr {
constexpr int D = 128;
constexpr int KS = D / 16;       // S-MFMA k-steps
constexpr int DB = D / 32;       // O^T row blocks
constexpr int TK = 64;           // KV positions per KV tile
constexpr int MAXK = 8;          // KV tiles in LDS: n_kv <= 512
constexpr int NW = 8;            // wavefronts
constexpr int NT = 64 * NW;
constexpr int ROW = D * 2;       // bytes per f16 row
constexpr int VT = TK * ROW;     // one V tile (16 KiB)
constexpr int QT = 32 * ROW;     // one staged query tile (8 KiB)
constexpr int NE = 16 * DB;      // O elements per lane
}  // namespace pr

// A barrier that orders LDS accesses only (a full __syncthreads() would also
// wait for every global load still in flight).
__device__ __forceinline__ void pr_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// MM 1: mask tensor, 2: implicit mask, 3: mask tensor with the live interval
// of each mask row found by a pre-pass (a.mask_rows; see mask_rows_kernel)
template <int MM, bool QF16>
__global__ __launch_bounds__(pr::NT) void fa_prefill_pair(AttnArgs a, GridMap gm, DivMod hmd, DivMod bmd, int nt,
                                                           int nk) {
    using namespace pr;
    static_assert(MM == 1 || MM == 2 || MM == 3, "masked calls only");
    constexpr bool TENSOR = MM == 1 || MM == 3;   // mixed blocks read their mask words from the tensor
    __shared__ __attribute__((aligned(16))) char sV[MAXK * VT];   // V tiles; then the published O
    __shared__ __attribute__((aligned(16))) char sQ[2 * QT];      // query tiles A (slot 0), B (slot 1)
    __shared__ float s_ml[2 * NW * 64];                           // published m, then l
    __shared__ uint8_t s_cls[2 * MAXK];                           // classes of (A, j), then (B, j)
    static_assert(NW * NE * 64 * 4 <= MAXK * VT, "published O fits the V area");

    int p, h, b, hk, bkv;
    gm.locate(blockIdx.x, p, h, b, hk, bkv);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 31;
    const int hh = lane >> 5;
    const int tA = p, tB = nt - 1 - p;
    const bool hasA = tA < tB;
    const char* kb = (const char*)a.k + (int64_t)hk * a.k_nb2 + (int64_t)bkv * a.k_nb3;
    const char* vb = (const char*)a.v + (int64_t)hk * a.v_nb2 + (int64_t)bkv * a.v_nb3;
    const float c = a.scale_log2;

    // ---- mask words of block (T, j) for this lane ----------------------------
    // Row 32 T + nl; element 2 w + e of 32-block kvb is half e of mw[kvb][w].
    // Lane half 0 holds positions 0..15 of each 32-block in order, half 1
    // positions 16..31 with its two 8-position halves swapped (the row-to-KV
    // permutation). Positions past n_kv and rows past n_q read -inf.
    // Mask rows of query tile T are addressed from a 16-byte-aligned scalar
    // base (the tile's first row rounded down) by 32-bit offsets: row rr of
    // the tile starts rs = d0 + rr * m_nb1 bytes after it (the host keeps
    // n_q * m_nb1 below 2^31 and m_nb1 below 2^24). Rows past n_q read the
    // tile's first row (their entries are dropped).
    const char* mplane = nullptr;
    if constexpr (TENSOR)
        mplane = (const char*)a.mask + (int64_t)hmd.mod((uint32_t)h) * a.m_nb2 + (int64_t)bmd.mod((uint32_t)b) * a.m_nb3;
    const uint32_t mnb = (uint32_t)a.m_nb1;
    const uint32_t rowbytes = 2u * (uint32_t)a.nkv;   // bytes of mask data per row
    auto mtile = [&](int T, uint32_t& d0) -> const char* {
        const uintptr_t t0 = reinterpret_cast<uintptr_t>(mplane) + (uintptr_t)(32 * T) * (uintptr_t)a.m_nb1;
        d0 = (uint32_t)(t0 & 15);
        return reinterpret_cast<const char*>(t0 - d0);
    };
    // Tensor: the lane's 16 entries of a 32-block are 32 bytes at any 2-byte
    // alignment (voxtral's n x n rows are 2n bytes apart), read as the three
    // 16-byte-aligned chunks that cover them. A chunk past the row's last data
    // granule is replaced by that granule, so every chunk read holds mask data
    // of the row (same allocation, same page); entries taken from it lie past
    // n_kv and are replaced by -inf.
    auto mw_rs = [&](int T, uint32_t d0) {   // start of the lane's row, from the tile base
        const int rr = 32 * T + nl < a.nq ? nl : 0;
        return d0 + __umul24((uint32_t)rr, mnb);
    };
    auto mw_issue = [&](int T, int j, u32x4 (&ch)[2][3]) {
        uint32_t d0;
        const char* mb = mtile(T, d0);
        const uint32_t rs = mw_rs(T, d0);
        const uint32_t last = (rs + rowbytes - 1u) & ~15u;
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb) {
            const uint32_t pa = (rs + 2u * (uint32_t)(TK * j + 32 * kvb + 16 * hh)) & ~15u;
            const int lim = (int)(last - pa);   // a multiple of 16
#pragma unroll
            for (int i = 0; i < 3; ++i) ch[kvb][i] = *(const u32x4*)(mb + (pa + (uint32_t)min(16 * i, lim)));
        }
    };
    auto mw_finish = [&](int T, int j, const u32x4 (&ch)[2][3], uint32_t (&mw)[2][8]) {
        const int row = 32 * T + nl;
        uint32_t d0;
        (void)mtile(T, d0);
        const uint32_t rs = mw_rs(T, d0);
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb) {
            const int sh = (int)((rs + 2u * (uint32_t)(TK * j + 32 * kvb + 16 * hh)) & 15u);
            const int q4 = sh >> 2, s2 = sh & 2;
            uint32_t d[12];
#pragma unroll
            for (int i = 0; i < 3; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) d[4 * i + k] = ch[kvb][i][k];
            uint32_t e[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) e[k] = q4 == 0 ? d[k] : q4 == 1 ? d[k + 1] : q4 == 2 ? d[k + 2] : d[k + 3];
            uint32_t wv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) wv[k] = __builtin_amdgcn_alignbyte(e[k + 1], e[k], (uint32_t)s2);
#pragma unroll
            for (int w = 0; w < 8; ++w) mw[kvb][w] = hh ? wv[(w + 4) & 7] : wv[w];
        }
        if (row >= a.nq) {
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int w = 0; w < 8; ++w) mw[kvb][w] = 0xFC00FC00u;
        } else if (TK * j + TK > a.nkv) {
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int w = 0; w < 8; ++w)
#pragma unroll
                    for (int e2 = 0; e2 < 2; ++e2)
                        if (TK * j + 32 * kvb + pf_kv_of(hh, 2 * w + e2) >= a.nkv)
                            mw[kvb][w] = (mw[kvb][w] & (0xFFFF0000u >> (16 * e2))) | (0xFC00u << (16 * e2));
        }
    };
    // Implicit: 0 where row attends kv, -inf elsewhere (rows past n_q use row
    // 0, as the tensor path of fa_prefill.hip does; they are never stored).
    auto mw_formula = [&](int T, int j, uint32_t (&mw)[2][8]) {
        const int row = 32 * T + nl;
        const int64_t lastc = (int64_t)(row < a.nq ? row : 0) + a.im_offset;
        const int64_t firstc = a.im_window > 0 ? lastc - a.im_window + 1 : INT64_MIN;
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                uint32_t pair = 0;
#pragma unroll
                for (int e2 = 0; e2 < 2; ++e2) {
                    const int kv = TK * j + 32 * kvb + pf_kv_of(hh, 2 * w + e2);
                    const bool live = kv < a.nkv && (int64_t)kv <= lastc && (int64_t)kv >= firstc;
                    pair |= (live ? 0u : (uint32_t)kF16NegInf) << (16 * e2);
                }
                mw[kvb][w] = pair;
            }
    };
    // MM 3, from the row's interval {lo, hi} ({n_kv, -1}: no live entry)
    auto mw_interval = [&](int j, int2 ivl, uint32_t (&mw)[2][8]) {
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                uint32_t pair = 0;
#pragma unroll
                for (int e2 = 0; e2 < 2; ++e2) {
                    const int kv = TK * j + 32 * kvb + pf_kv_of(hh, 2 * w + e2);
                    const bool live = kv < a.nkv && kv >= ivl.x && kv <= ivl.y;
                    pair |= (live ? 0u : (uint32_t)kF16NegInf) << (16 * e2);
                }
                mw[kvb][w] = pair;
            }
    };
    // class of block (T, j) from the formula: 0 dead, 1 every entry 0, 3 mixed
    // (a KV tile running past n_kv is mixed)
    auto cls_formula = [&](int T, int j) -> int {
        const int64_t r0 = 32 * T, r1 = (int64_t)min(32 * T + 32, a.nq) - 1;
        const int64_t c0 = TK * j, c1 = (int64_t)min(TK * j + TK, a.nkv) - 1;
        if (r1 < r0 || c1 < c0) return 0;
        const int64_t off = a.im_offset, W = a.im_window;
        if (c0 > r1 + off || (W > 0 && c1 < r0 + off - W + 1)) return 0;
        const bool all = c1 <= r0 + off && (W == 0 || c0 >= r1 + off - W + 1);
        return (all && TK * j + TK <= a.nkv) ? 1 : 3;
    };

    // ---- Q loads of both tiles (rows past n_q load row n_q - 1, zeroed when
    // staged; no load sits under a branch). Q is read once: nontemporal loads
    // (12.8 -> 12.3 us per layer at 439 causal; nontemporal output stores of
    // 32-byte row pieces measured slower) -----------------------------------------
    constexpr int QCH = QF16 ? 16 : 32;           // 16-byte global chunks per row
    constexpr int QPT = 2 * 32 * QCH / NT;        // per thread
    floatx4 qraw[QPT];
    int rowpos = 0;   // rotary position of staged row `lane` (0-31 tile A, 32-63 tile B; F32 Q)
    // (rows from a scalar base by 32-bit offsets: the host keeps n_q * q_nb1
    // below 2^31 and q_nb1 below 2^24)
    const char* qhb = (const char*)a.q + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
    const int* qpb = a.rope_pos ? a.rope_pos + (int64_t)b * a.nq : (const int*)a.q;
    auto issue_q = [&]() {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int i = tid + NT * u;
            const int s = i / (32 * QCH), r = (i / QCH) % 32, cch = i % QCH;
            const int row = min(32 * (s ? tB : tA) + r, a.nq - 1);
            qraw[u] = __builtin_nontemporal_load(
                (const floatx4*)(qhb + (__umul24((uint32_t)row, (uint32_t)a.q_nb1) + (uint32_t)(cch * 16))));
        }
        if constexpr (!QF16) {
            // read without a branch: without a rotary embedding it reads the
            // first word of Q, unused
            const int rrow = min(32 * (lane >= 32 ? tB : tA) + (lane & 31), a.nq - 1);
            rowpos = qpb[(uint32_t)(a.rope_pos ? rrow : 0)];
        }
    };

    // ---- classes of the pair's blocks ------------------------------------------
    // candidates of this wavefront (mask tensor): (B, wave) and (A, 7 - wave)
    const int jB = wave, jA = MAXK - 1 - wave;
    const bool candB = jB < nk, candA = hasA && jA < nk;
    uint32_t liveA = 0, liveB = 0, mixA = 0, mixB = 0;
    int2 iv = {0, 0};                       // MM 3: the interval of row 32 T + (lane % 32), T = A / B by lane half
    bool ivA = false, ivB = false;          // MM 3: every real row of tile A / B is an interval (or empty)
    if constexpr (MM == 1) {
        // A candidate's 32 rows are read as the 16-byte-aligned chunks that
        // cover each row's 128-byte segment: nine lanes per row (lane 63
        // idle), seven rows per load, five loads. A chunk past the row's last
        // data granule is replaced by that granule; entries outside the
        // segment, past n_kv or of rows past n_q are dropped in registers.
        const int lr = lane / 9, lc = lane - 9 * (lane / 9);
        // e0[u]: entry index (in the row) of the lane's chunk's first entry,
        // or a large value for a lane without a row (no entry is taken)
        auto cls_issue = [&](int T, int j, u32x4 (&cw)[5], int (&e0)[5]) {
            uint32_t d0;
            const char* mb = mtile(T, d0);
#pragma unroll
            for (int u = 0; u < 5; ++u) {
                const int rr = 7 * u + lr;
                const bool ok = lr < 7 && rr < 32 && 32 * T + rr < a.nq;
                const uint32_t rs = d0 + (ok ? __umul24((uint32_t)rr, mnb) : 0u);
                const uint32_t last = (rs + rowbytes - 1u) & ~15u;
                const uint32_t pa = (rs + 2u * TK * (uint32_t)j) & ~15u;
                const int lim = (int)(last - pa);
                cw[u] = *(const u32x4*)(mb + (pa + (uint32_t)min(16 * lc, lim)));
                e0[u] = ok ? ((int)(pa - rs) + 16 * lc) / 2 : (1 << 20);
            }
        };
        auto cls_eval = [&](int j, const u32x4 (&cw)[5], const int (&e0)[5]) -> int {
            bool live = false, nonzero = false;
#pragma unroll
            for (int u = 0; u < 5; ++u) {
                // entries k of the chunk inside [64 j, min(64 j + 64, n_kv))
                const int lo = max(TK * j - e0[u], 0), hi = min(min(TK * j + TK, a.nkv) - e0[u], 8);
                const uint32_t m8 = hi > lo ? (((1u << hi) - 1u) & ~((1u << lo) - 1u)) : 0u;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t wm = (((m8 >> (2 * w)) & 1u) ? 0x0000FFFFu : 0u) |
                                        (((m8 >> (2 * w + 1)) & 1u) ? 0xFFFF0000u : 0u);
                    live |= ((cw[u][w] ^ 0xFC00FC00u) & wm) != 0u;
                    nonzero |= (cw[u][w] & 0x7FFF7FFFu & wm) != 0u;
                }
            }
            const bool any_live = __any(live);
            // a KV tile running past n_kv is mixed (its positions there are -inf)
            return !any_live ? 0 : (__any(nonzero) || TK * j + TK > a.nkv) ? 3 : 1;
        };
        u32x4 cwB[5], cwA[5];
        int e0B[5], e0A[5];
        // (a candidate that does not exist reads tile B's or A's first block)
        cls_issue(tB, candB ? jB : 0, cwB, e0B);
        cls_issue(tA, candA ? jA : 0, cwA, e0A);
        issue_q();   // after the mask loads: their wait does not include Q's
        const int cB = cls_eval(candB ? jB : 0, cwB, e0B), cA = cls_eval(candA ? jA : 0, cwA, e0A);
        if (lane == 0) {
            if (candB) s_cls[MAXK + jB] = (uint8_t)cB;
            if (candA) s_cls[jA] = (uint8_t)cA;
        }
        pr_lds_barrier();
    } else if constexpr (MM == 3) {
        // Classes from the rows' intervals, with no mask reads and no barrier:
        // lane l holds row 32 T + (l % 32) of tile T = A (l < 32) or B. Per
        // block j (positions [64 j, 64 j + 64) within n_kv) a row is live when
        // its interval meets the block and covers it when it holds all of it;
        // a row that is not an interval makes every block of its tile live and
        // mixed (its words then come from the tensor, correct for any mask),
        // an empty row makes none live and none covered, a row past n_q (or of
        // a missing tile A) counts as covering and not live. Ballots over each
        // half of the wavefront give the tile's live and mixed blocks.
        const int2* tab = a.mask_rows + ((int64_t)bmd.mod((uint32_t)b) * a.hm + hmd.mod((uint32_t)h)) * a.nq;
        const int Tl = lane < 32 ? tA : tB;
        const int rowl = 32 * Tl + nl;
        iv = tab[min(rowl, a.nq - 1)];   // unconditional: no wait at a join
        issue_q();   // after the interval load: its wait does not include Q's
        const bool realrow = rowl < a.nq && (lane >= 32 || hasA);
        const uint64_t bad = __ballot(realrow && iv.x == -2);
        ivA = (uint32_t)bad == 0u;
        ivB = (uint32_t)(bad >> 32) == 0u;
        uint32_t lv = 0, cv = 0;
#pragma unroll
        for (int j = 0; j < MAXK; ++j) {
            const int c0 = TK * j, c1 = min(TK * j + TK, a.nkv) - 1;
            const bool inb = j < nk;
            const bool meets = iv.x <= c1 && iv.y >= c0;       // false for an empty row {n, -1}
            const bool holds = iv.x <= c0 && iv.y >= c1 && iv.x >= 0;
            const bool live = inb && (iv.x == -2 || meets);
            const bool cov = iv.x != -2 && holds;
            lv |= (realrow && live ? 1u : 0u) << j;
            cv |= (!realrow || cov ? 1u : 0u) << j;
        }
#pragma unroll
        for (int j = 0; j < MAXK; ++j) {
            const uint64_t bl = __ballot((lv >> j) & 1u), bc = __ballot(!((cv >> j) & 1u));
            const uint32_t la = (uint32_t)bl != 0u, lb = (uint32_t)(bl >> 32) != 0u;
            // a KV tile running past n_kv is mixed (its positions there are -inf)
            const uint32_t fa = (uint32_t)bc == 0u && TK * j + TK <= a.nkv;
            const uint32_t fb = (uint32_t)(bc >> 32) == 0u && TK * j + TK <= a.nkv;
            liveA |= la << j;
            liveB |= lb << j;
            mixA |= (la & (fa ^ 1u)) << j;
            mixB |= (lb & (fb ^ 1u)) << j;
        }
    } else {
        issue_q();
    }
    // Lane L < 16 takes block (A, L) or (B, L - 8) and two ballots form the
    // masks (a loop over the blocks in every wavefront compiled to ~500
    // dependent scalar and branch instructions: 1.7 us).
    if constexpr (MM != 3) {
        const int lc = lane & 15;
        const int jl = lc & (MAXK - 1);
        const bool onb = lc >= MAXK;
        int k = 0;
        if (lane < 2 * MAXK && jl < nk && (onb || hasA)) {
            if constexpr (MM == 1) k = s_cls[lc];
            else k = cls_formula(onb ? tB : tA, jl);
        }
        const uint64_t lv = __ballot(k != 0), mx = __ballot(k == 3);
        liveA = (uint32_t)lv & 0xFFu;
        liveB = (uint32_t)(lv >> MAXK) & 0xFFu;
        mixA = (uint32_t)mx & 0xFFu;
        mixB = (uint32_t)(mx >> MAXK) & 0xFFu;
    }

    // ---- assignment ------------------------------------------------------------
    const int nA = __builtin_popcount(liveA), nB = __builtin_popcount(liveB);
    int wB = NW;
    if (hasA) {
        if (nA + nB == 0) wB = NW / 2;
        else wB = min(max((NW * nB + (nA + nB) / 2) / (nA + nB), 1), NW - 1);
    }
    const bool onB = wave < wB;
    const int T = onB ? tB : tA;
    const int wT = onB ? wB : NW - wB;             // wavefronts of this tile
    const int iT = onB ? wave : NW - 1 - wave;     // index among them
    const uint32_t live = onB ? liveB : liveA;
    const uint32_t mix = onB ? mixB : mixA;
    const int nT = onB ? nB : nA;
    const int nblk = nT > iT ? (nT - iT + wT - 1) / wT : 0;
    // KV tile of this wavefront's k-th block: the (iT + k wT)-th live tile
    auto block_tile = [&](int k) -> int {
        uint32_t m = live;
        for (int r = iT + k * wT; r > 0; --r) m &= m - 1;   // drop the lowest set bits
        return m ? __builtin_ctz(m) : 0;
    };

    // ---- the wavefront's blocks (at most two) and their mask words ----------
    // (mask tensor: the words of a mixed block in the accumulator layout are
    // read here and finished after the wait below; implicit: the formula)
    const int j0 = nblk > 0 ? block_tile(0) : 0;
    const int j1 = nblk > 1 ? block_tile(1) : 0;
    const bool mix0 = nblk > 0 && ((mix >> j0) & 1u);
    const bool mix1 = nblk > 1 && ((mix >> j1) & 1u);
    uint32_t mw0[2][8], mw1[2][8];
    u32x4 chr0[2][3], chr1[2][3];
    // MM 3: a tile whose rows are all intervals forms its mixed blocks' words
    // from the lane's row interval (the row's lane in the classification
    // layout is nl for tile A, 32 + nl for tile B); any other tile reads them
    // from the tensor
    bool mw_tensor = TENSOR;
    int2 ivr = {0, 0};
    if constexpr (MM == 3) {
        mw_tensor = !(onB ? ivB : ivA);
        const int src = (onB ? 32 : 0) + nl;
        ivr.x = __shfl(iv.x, src, 64);
        ivr.y = __shfl(iv.y, src, 64);
    }
    if (mix0) {
        if (mw_tensor) mw_issue(T, j0, chr0);
        else if constexpr (MM == 3) mw_interval(j0, ivr, mw0);
        else mw_formula(T, j0, mw0);
    }
    if (mix1) {
        if (mw_tensor) mw_issue(T, j1, chr1);
        else if constexpr (MM == 3) mw_interval(j1, ivr, mw1);
        else mw_formula(T, j1, mw1);
    }

    // ---- K, then V: every live KV tile of the pair through one LDS area -----
    // Tile j's rows 4 g .. 4 g + 3 (g = 0..15) are one copy instruction;
    // wavefront w issues g = w and w + 8 of every tile. Lane l writes LDS
    // chunk l % 16 of row 4 g + l / 16, which holds the row's chunk
    // (l % 16) ^ swizzle(row) (the K or the V swizzle). Rows past n_kv repeat
    // row n_kv - 1.
    const uint32_t used = liveA | liveB;
    const uint32_t lds_kv = lds_offset(sV);
    const int rl = lane >> 4;
    auto issue_tiles = [&](const char* base, int64_t nb1, auto is_k) {
        for (int jt = 0; jt < nk; ++jt) {
            if (!((used >> jt) & 1u)) continue;
            const int kv0 = TK * jt;
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
                const int g = wave + NW * gg;
                const int r = 4 * g + rl;
                const int col = ((lane & 15) ^ (decltype(is_k)::value ? swz_k<D>(r) : swz_v<D>(r))) * 16;
                const uint32_t dst = lds_kv + jt * VT + 4 * g * ROW;
                if (kv0 + TK <= a.nkv) {
                    dma16(base + (int64_t)kv0 * nb1, (uint32_t)r * (uint32_t)nb1 + col, dst);
                } else {
                    const int kv = min(kv0 + r, a.nkv - 1);
                    dma16_addr(base + (int64_t)kv * nb1 + col, dst);
                }
            }
        }
    };
    issue_tiles(kb, a.k_nb1, std::true_type{});

    // ---- Q: wait for every load, round to f16, stage -------------------------
    wait_all_mem();
    if (mw_tensor) {
        if (mix0) mw_finish(T, j0, chr0, mw0);
        if (mix1) mw_finish(T, j1, chr1, mw1);
    }
    // Rotary angles (F32 Q with rope_pos): the angle of pair j of staged row
    // R (0-31 tile A, 32-63 tile B) in a table over the Q area, at float
    // R * 64 + (j ^ R) (the XOR spreads the writes, one pair of every row,
    // and the reads, two pairs of one row, over the banks). Wavefront 0 forms
    // each row's running product once (lane = row), as ggml builds its
    // cos / sin cache, and every lane takes the cos / sin of its chunk's two
    // pairs from it (a per-lane product loop cost ~6 instructions per step
    // for up to 62 steps per chunk).
    float2 qcs[QPT][2];
    if constexpr (!QF16) {
        if (a.rope_pos) {
            float* tab = reinterpret_cast<float*>(sQ);
            static_assert(64 * (D / 2) * sizeof(float) <= 2 * QT, "angle table fits the Q area");
            if (wave == 0) {
                float th = (float)rowpos;
#pragma unroll
                for (int j = 0; j < D / 2; ++j) {
                    tab[lane * 64 + (j ^ lane)] = th;
                    th *= a.rope_ts;
                }
            }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < QPT; ++u) {
                const int i = tid + NT * u;
                const int s = i / (32 * QCH), r = (i / QCH) % 32, cch = i % QCH;
                const int R = 32 * s + r;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int j = 2 * cch + k;
                    qcs[u][k] = rope_cs_of_angle(tab[R * 64 + (j ^ R)]);
                }
            }
            __syncthreads();   // every angle read before the rows overwrite the table
        }
    }
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int i = tid + NT * u;
        const int s = i / (32 * QCH), r = (i / QCH) % 32, cch = i % QCH;
        floatx4 x = qraw[u];
        if (32 * (s ? tB : tA) + r >= a.nq) x = floatx4{0.f, 0.f, 0.f, 0.f};
        char* qrow = sQ + s * QT + r * ROW;
        if constexpr (QF16) {
            *(floatx4*)(qrow + ((cch ^ (r & 15)) * 16)) = x;
        } else {
            // rotated first when a rotary embedding is given (ggml rotates
            // Q before the attention node)
            float xr[4] = {x[0], x[1], x[2], x[3]};
            if (a.rope_pos) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    if (4 * cch + 2 * k < a.rope_dims) {
                        const float cs_ = qcs[u][k].x, sn = qcs[u][k].y;
                        const float x0 = xr[2 * k], x1 = xr[2 * k + 1];
                        xr[2 * k] = x0 * cs_ - x1 * sn;
                        xr[2 * k + 1] = x0 * sn + x1 * cs_;
                    }
                }
            }
            half4 v;
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) v[e2] = (_Float16)xr[e2];
            *(half4*)(qrow + (((cch >> 1) ^ (r & 15)) * 16) + (cch & 1) * 8) = v;
        }
    }
    __syncthreads();   // Q staged, K tiles visible

    // ---- S^T = K Q^T of the wavefront's blocks, K operands from LDS ----------
    // (A-operand row nl of 32-block kvb is K row krow of it, chunk 2 ks + hh)
    int kaddr[KS];
    {
        const int am = nl >> 3, ahb = (nl >> 2) & 1, ab = nl & 3;
        const int krow = ahb ? 16 + ((am + 2) & 3) * 4 + ab : 4 * am + ab;
        const int kx = hh ^ swz_k<D>(krow);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kaddr[ks] = krow * ROW + ((2 * ks) ^ kx) * 16;
    }
    const char* qs = sQ + (onB ? QT : 0) + nl * ROW;
    floatx16 S0[2], S1[2];
    auto s_block = [&](int jt, floatx16 (&S)[2]) {
        const char* kt = sV + jt * VT;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const half8 qk = *(const half8*)(qs + (((2 * ks + hh) ^ (nl & 15)) * 16));
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb) {
                const half8 kk = *(const half8*)(kt + kaddr[ks] + 32 * kvb * ROW);
                S[kvb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kk, qk, ks == 0 ? floatx16{} : S[kvb], 0, 0, 0);
            }
        }
    };
    if (nblk > 0) s_block(j0, S0);
    if (nblk > 1) s_block(j1, S1);
    __syncthreads();   // every K read done: the area takes the V tiles
    issue_tiles(vb, a.v_nb1, std::false_type{});

    // ---- softmax over the wavefront's blocks (while V lands) ------------------
    // scores in log2 units with the mask added (-inf stays -inf); one max over
    // both blocks, so O needs no rescale
    auto scores = [&](floatx16 (&S)[2], bool mixed, const uint32_t (&mwx)[2][8]) -> float {
        float mx = -INFINITY;
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                float x = S[kvb][jj] * c;
                if (mixed) {
                    const half2 m2 = __builtin_bit_cast(half2, mwx[kvb][jj >> 1]);
                    x = fmaf((float)m2[jj & 1], kLog2e, x);
                }
                S[kvb][jj] = x;
                mx = fmaxf(mx, x);
            }
        return mx;
    };
    float mx = -INFINITY;
    if (nblk > 0) mx = scores(S0, mix0, mw0);
    if (nblk > 1) mx = fmaxf(mx, scores(S1, mix1, mw1));
    const float m_run = pair32_max(mx);
    const float ms = (m_run == -INFINITY) ? 0.f : m_run;
    const half2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    half8 P0[4], P1[4];
    float ls[2] = {0.f, 0.f};
    auto probs = [&](const floatx16 (&S)[2], half8 (&P)[4]) {
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {
            const int kvb = pc >> 1, cc = pc & 1;
#pragma unroll
            for (int i2 = 0; i2 < 8; ++i2) P[pc][i2] = (_Float16)exp2_fast(S[kvb][8 * cc + i2] - ms);
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const half2 p2 = {P[pc][2 * i2], P[pc][2 * i2 + 1]};
                ls[i2 & 1] = __builtin_amdgcn_fdot2(p2, ones, ls[i2 & 1], false);
            }
        }
    };
    if (nblk > 0) probs(S0, P0);
    if (nblk > 1) probs(S1, P1);
    const float l_run = ls[0] + ls[1];
    wait_all_mem();
    __syncthreads();   // V tiles visible

    // ---- O^T = V^T P^T -------------------------------------------------------
    floatx16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = floatx16{};
    const int vq = (lane & 15) >> 2;
    const int clo = 2 * ((lane & 31) >> 4) + ((lane & 3) >> 1);
    int vaddr[2][DB];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int db = 0; db < DB; ++db)
            vaddr[cc][db] = ((hh ? 24 - 8 * cc : 8 * cc) + vq) * ROW + ((4 * db + clo) ^ swz_v<D>(vq)) * 16 +
                            (lane & 1) * 8;
    auto pv_block = [&](int jt, const half8 (&P)[4]) {
        const char* vt = sV + jt * VT;
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {
            const int kvb = pc >> 1, cc = pc & 1;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const char* vp = vt + vaddr[cc][db] + 32 * kvb * ROW;
                const half4 lo4 = lds_read_tr16(vp);
                const half4 hi4 = lds_read_tr16(vp + 4 * ROW);
                const half8 va = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, P[pc], o[db], 0, 0, 0);
            }
        }
    };
    if (nblk > 0) pv_block(j0, P0);
    if (nblk > 1) pv_block(j1, P1);

    // ---- merge each tile over its wavefronts, normalise, store ---------------
    // Output group q = 4 db + a4 of a lane is accumulator quad a4 of O^T block
    // db: dims 32 db + 8 a4 + 4 hh .. + 3 of row 32 T + nl. A wavefront whose
    // tile has other wavefronts publishes its 16 groups as 16-byte chunks
    // (group q of lane l at float 4 (64 q + l) of its 16 KiB) with its m and l;
    // the tile's wavefronts then each merge groups iT, iT + wT, ... over all
    // of them, in wavefront order. A tile with one wavefront stores its own.
    const int row = 32 * T + nl;
    float* out_row = a.dst + (((int64_t)b * a.nq + (row < a.nq ? row : 0)) * a.hq + h) * D + 4 * hh;
    __syncthreads();   // every V read done: the V area takes the published O
    if (wT > 1) {
        floatx4* pub = (floatx4*)sV + wave * (16 * 64) + lane;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int db = q >> 2, a4 = q & 3;
            pub[q * 64] = floatx4{o[db][4 * a4], o[db][4 * a4 + 1], o[db][4 * a4 + 2], o[db][4 * a4 + 3]};
        }
        s_ml[wave * 64 + lane] = m_run;
        s_ml[NW * 64 + wave * 64 + lane] = l_run;
    }
    __syncthreads();
    if (wT == 1) {
        const float lt = pair32_sum(l_run);
        const float inv = (lt == 0.f) ? 0.f : 1.0f / lt;
        if (row < a.nq) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int db = q >> 2, a4 = q & 3;
                *(floatx4*)(out_row + 32 * db + 8 * a4) =
                    floatx4{o[db][4 * a4] * inv, o[db][4 * a4 + 1] * inv, o[db][4 * a4 + 2] * inv,
                            o[db][4 * a4 + 3] * inv};
            }
        }
    } else {
        // the tile's wavefronts: B's are 0 .. wB - 1, A's wB .. NW - 1; slots
        // past wT repeat the last one with weight 0
        const int g0 = onB ? 0 : wB;
        float mg[NW], lg[NW];
#pragma unroll
        for (int gi = 0; gi < NW; ++gi) {
            const int g = g0 + min(gi, wT - 1);
            mg[gi] = s_ml[g * 64 + lane];
            lg[gi] = s_ml[NW * 64 + g * 64 + lane];
        }
        float M = -INFINITY;
#pragma unroll
        for (int gi = 0; gi < NW; ++gi) M = fmaxf(M, mg[gi]);
        const float Ms = (M == -INFINITY) ? 0.f : M;
        float wg[NW];
        float lsum = 0.f;
#pragma unroll
        for (int gi = 0; gi < NW; ++gi) {
            wg[gi] = gi < wT ? exp2_fast(mg[gi] - Ms) : 0.f;
            lsum = fmaf(wg[gi], lg[gi], lsum);
        }
        const float lt = pair32_sum(lsum);
        const float inv = (lt == 0.f) ? 0.f : 1.0f / lt;
#pragma unroll
        for (int gi = 0; gi < NW; ++gi) wg[gi] *= inv;
        const floatx4* src = (const floatx4*)sV + lane;
        for (int q = iT; q < 16; q += wT) {
            floatx4 part[NW];
#pragma unroll
            for (int gi = 0; gi < NW; ++gi) part[gi] = src[(g0 + min(gi, wT - 1)) * (16 * 64) + q * 64];
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int gi = 0; gi < NW; ++gi)
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) acc[e2] = fmaf(wg[gi], part[gi][e2], acc[e2]);
            if (row < a.nq) *(floatx4*)(out_row + 32 * (q >> 2) + 8 * (q & 3)) = acc;
        }
    }
}

// Short masked prefill: hd 128, a mask tensor or an implicit mask, n_kv <= 512
// (a rotary embedding of F32 Q applied as it is staged).
// The 32-bit offsets of the kernel: Q and mask rows from a per-tile base
// (row strides below 2^24 bytes, n_q rows below 2^31 bytes).
bool prefill_pair_fits(const AttnArgs& a) {
    const int64_t lim = (int64_t)1 << 31, s24 = (int64_t)1 << 24;
    if (a.nq <= 0 || a.nq >= (1 << 24)) return false;
    if (a.q_nb1 < 0 || a.q_nb1 >= s24 || (int64_t)a.nq * a.q_nb1 >= lim) return false;
    if (a.mask && (a.m_nb1 < 0 || a.m_nb1 >= s24 || ((int64_t)a.nq + 32) * a.m_nb1 >= lim)) return false;
    return true;
}

hipError_t launch_prefill_pair(const AttnArgs& a, hipStream_t st) {
    using namespace pr;
    if (!(a.mask != nullptr || a.im_causal) || (a.rope_pos != nullptr && a.q_f16)) return hipErrorInvalidValue;
    const int nt = (a.nq + 31) / 32;
    const int nk = (a.nkv + TK - 1) / TK;
    if (nt <= 0 || nk <= 0 || nk > MAXK) return hipErrorInvalidValue;
    const int np = (nt + 1) / 2;
    const int64_t nwg = (int64_t)np * a.hq * a.b;
    if (nwg <= 0 || nwg > 0x7fffffff) return hipErrorInvalidValue;
    if (!prefill_pair_fits(a)) return hipErrorInvalidValue;
    const GridMap gm = GridMap::make((int)nwg, np, a.hq, a.hkv, a.b, a.bk);
    const DivMod hmd = DivMod::make(a.hm > 0 ? a.hm : 1), bmd = DivMod::make(a.bm > 0 ? a.bm : 1);
    const dim3 grid((unsigned)nwg), block(NT);
    if (a.im_causal) {
        if (a.q_f16) hipLaunchKernelGGL((fa_prefill_pair<2, true>), grid, block, 0, st, a, gm, hmd, bmd, nt, nk);
        else hipLaunchKernelGGL((fa_prefill_pair<2, false>), grid, block, 0, st, a, gm, hmd, bmd, nt, nk);
    } else if (a.mask_rows) {
        if (a.q_f16) hipLaunchKernelGGL((fa_prefill_pair<3, true>), grid, block, 0, st, a, gm, hmd, bmd, nt, nk);
        else hipLaunchKernelGGL((fa_prefill_pair<3, false>), grid, block, 0, st, a, gm, hmd, bmd, nt, nk);
    } else {
        if (a.q_f16) hipLaunchKernelGGL((fa_prefill_pair<1, true>), grid, block, 0, st, a, gm, hmd, bmd, nt, nk);
        else hipLaunchKernelGGL((fa_prefill_pair<1, false>), grid, block, 0, st, a, gm, hmd, bmd, nt, nk);
    }
    return hipGetLastError();
}

}  // namespace vxfa
