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
//   [32 qw, 32 qw + 32) of the block and the kg-th 64-position tile of every
//   KV step of BS = 64 * KVG positions. With hd 64 a workgroup has 16
//   wavefronts, 4 per SIMD, so while some run their softmax (VALU) the
//   others keep the matrix pipe busy. The KVG partial results are merged
//   through LDS at the end (log-sum-exp).
//   The 1-D grid is mapped so the workgroups that share one head's K/V are
//   dispatched to the same XCD (workgroups are dealt to the 8 XCDs round
//   robin), keeping that head's K/V in one L2. Without a mask each workgroup
//   starts its KV walk at a step set by its query block, so the workgroups of
//   one head do not all miss on the same tile at once.
// Pipeline: K/V steps are double buffered in LDS and filled straight from
//   global memory with global_load_lds_dwordx4 (no staging registers), the
//   next step streaming in while the current one is computed; one barrier
//   per step. The loads are issued through inline assembly: the compiler
//   then neither orders the reads of one stage after the loads into the
//   other (it cannot tell the stages apart inside one array) nor counts them,
//   and each wavefront waits for its own loads (s_waitcnt vmcnt(0)) right
//   before the step's barrier.
// LDS rows are unpadded, row-major [kv][d], with the 16-byte chunks of each
//   row XOR-swizzled: chunk c of row r sits at position c ^ f(r). Unswizzled,
//   the K-operand reads (16 rows, one chunk) hit the same banks 8-fold (hd 64)
//   or 16-fold (hd 128). Measured on gfx950 with 16 wavefronts per CU, these
//   f make the K reads (ds_read_b128) and the V^T reads (8-byte transposed
//   reads) conflict-free:
//     hd 64 :  K f(r) = (r ^ r >> 2) & 7,          V f(r) = (r & 2) << 1
//     hd 128:  K f(r) = (r >> 1 ^ r << 2) & 15,    V f(r) = (r & 3) << 2
//   None depends on row bits 5 and up, so rows 32 apart share the swizzle,
//   and the V swizzles depend on the row's position in its 4-row group only:
//   every LDS read address is a lane constant plus an immediate.
// MFMA layouts (v_mfma_f32_32x32x16_f16, lane = 32*hh + nl):
//   S^T = K Q^T: A = K rows from LDS (128-bit reads), B = Q (registers, f16
//     rounded like ggml's Q conversion). Lane (nl, hh) receives query row nl
//     and 16 KV positions of each 32-block, so the row max needs one
//     cross-lane step (v_permlane32_swap).
//   O^T = V^T P^T: B = P straight from the softmax registers (f16), A = V^T
//     fetched from the row-major V tile with ds_read_b64_tr_b16, which
//     transposes 16-bit elements across each 16-lane group.
// Softmax in fp32 with exp2 (scale*log2(e) folded into one FMA per score).
//   The running max is raised only when a tile's max exceeds it by more than
//   2^8, so the O rescale runs on few tiles; P then stays below 256 in f16.
// Row-to-KV mapping inside a 32-position block (lane half hh, accumulator
// element j, a = j / 4, b = j % 4):
//   hh = 0 : kv = 4a + b            hh = 1 : kv = 16 + 4((a + 2) & 3) + b
// so that each half of a lane's accumulator (j < 8, j >= 8) covers 8
// contiguous positions in increasing order, the order the P.V operand needs.
#include "fa_common.h"

#include <type_traits>

namespace vxfa {

constexpr int PF_BN = 64;                // KV positions per wavefront tile
constexpr float PF_TAU = 8.0f;

constexpr int PF_MAXT = 512;            // 64-position tiles classified per row group

// Tile classes of an additive mask over the workgroup's rows, for row group g
// (32 rows) and 64-position tile T: flags[g * PF_MAXT + T] has bit 0 set when
// some entry is not -inf and bit 1 when some entry is not +-0. So 1 = every
// entry is zero (the tile needs no mask values), 2 = every entry is -inf (the
// tile contributes nothing), 3 = mixed; a partial last tile with a live entry
// counts as mixed, and a group without rows reads 0 (nothing to do). Tiles
// from PF_MAXT on are not classified (read as mixed).
// Also returns the live range [lo, hi) rounded out to whole tiles, which
// selects the same KV steps as the exact range (steps are whole tiles).
//
// One wavefront takes one (group, tile) unit at a time, four units per
// batch, all of a batch's loads issued before any is used and none under a
// branch. A unit's rows are 128-byte segments at any 2-byte alignment
// (voxtral's n x n mask rows are 2n bytes apart): nine lanes read one row's
// segment as the 16-byte-aligned chunks that cover it, seven rows per load
// instruction, five instructions per unit. Rows 32 apart share their
// misalignment (the stride is even), so each lane sets up its five rows once:
// their aligned start, their last chunk holding mask data, and which entries of
// its chunk fall inside a full tile (all 8 but for the first and last chunk
// of the segment). A chunk past a row's data is replaced by the row's last
// one, and a lane without a row (or past the workgroup's rows) reads row 0,
// so every chunk read holds mask data: it lies in the same 16-byte granule of
// the same allocation and page. Entries outside the tile, or read in place of
// another, are dropped in registers.
__device__ __forceinline__ uint32_t half_mask(uint32_t m8, int j) {   // entries 2j, 2j+1 -> 16-bit halves
    return (((m8 >> (2 * j)) & 1u) ? 0x0000FFFFu : 0u) | (((m8 >> (2 * j + 1)) & 1u) ? 0xFFFF0000u : 0u);
}
__device__ __forceinline__ uint32_t entry_range(int e_lo, int e_hi) {   // bits [e_lo, e_hi) of 8
    return e_hi > e_lo ? (((1u << e_hi) - 1u) & ~((1u << e_lo) - 1u)) : 0u;
}
// A barrier that orders LDS accesses only: a full __syncthreads() would
// also wait for every global load still in flight (here, the query rows).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// after_loads() runs once per wavefront right after its first batch's loads
// are issued (before any is waited for): the caller issues its own loads
// there, so the scan's wait does not include them (loads complete in order).
template <int NT, int NG, class F>
__device__ __forceinline__ void mask_scan_tiles(const uint16_t* base, int64_t row_stride, int rows, int n,
                                                uint8_t* flags, int* red, int& lo, int& hi, F&& after_loads) {
    constexpr int NWV = NT / 64;
    constexpr int UB = 4;            // units per wavefront batch
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ntile_all = (n + 63) >> 6;
    const int ntile = min(ntile_all, PF_MAXT);
    const int units = NG * ntile;
    const int lr = lane / 9, lc = lane - 9 * lr;   // row in a batch of 7 (lane 63 idle), chunk 0..8
    const int last_span = n - 64 * (ntile_all - 1);   // entries of the last tile
    // (pointer arithmetic on const char*: integer addresses would make the
    // compiler fall back to flat loads)
    const char* b0 = reinterpret_cast<const char*>(base);
    const int64_t gstride = 32 * row_stride;
    // row 0 of the workgroup: the row read in place of a missing one
    const int mis0 = (int)(reinterpret_cast<uintptr_t>(b0) & 15);
    const char* rowa0 = b0 - mis0;
    const int kmax0 = (2 * n - 1 + mis0) >> 4;
    // this lane's row 7 bt + lr of group 0
    const char* rowa[5];   // 16-byte-aligned start
    int kmax[5];           // last chunk holding mask data
    int mis2[5];           // misalignment in entries
    uint32_t m8i[5];       // entries of the lane's chunk inside a full tile
    uint32_t hmi[5][4];    // the same as 16-bit halves of the chunk's words
#pragma unroll
    for (int bt = 0; bt < 5; ++bt) {
        const int rr = 7 * bt + lr;
        const bool lane_row = lr < 7 && rr < 32;
        const char* rp = b0 + (int64_t)(lane_row ? rr : 0) * row_stride;
        const int mis = (int)(reinterpret_cast<uintptr_t>(rp) & 15);
        rowa[bt] = rp - mis;
        kmax[bt] = (2 * n - 1 + mis) >> 4;
        mis2[bt] = mis >> 1;
        m8i[bt] = lane_row ? entry_range(lc == 0 ? mis >> 1 : 0, lc == 8 ? mis >> 1 : 8) : 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) hmi[bt][j] = half_mask(m8i[bt], j);
    }
    int tlo = 0x7fffffff, thi = -1;                // live tiles (wave-uniform)
    // The first batch is straight-line code, so no wait a loop's head would
    // get for loads issued earlier comes before its loads and Q's.
    auto batch = [&](int ub, bool first) {
        u32x4 w[UB][5];
        bool okr[UB][5];
#pragma unroll
        for (int i = 0; i < UB; ++i) {
            const int u = min(ub + i, units - 1);   // past the last unit: a repeat, unused
            const int g = u / ntile, t = u - g * ntile;
#pragma unroll
            for (int bt = 0; bt < 5; ++bt) {
                const int rr = 7 * bt + lr;
                const bool ok = lr < 7 && rr < 32 && 32 * g + rr < rows;
                const char* ra = ok ? rowa[bt] + (int64_t)g * gstride : rowa0;
                const int k = min(8 * t + lc, ok ? kmax[bt] : kmax0);
                okr[i][bt] = ok;
                w[i][bt] = *reinterpret_cast<const u32x4*>(ra + 16 * k);
            }
        }
        if (first) after_loads();
#pragma unroll
        for (int i = 0; i < UB; ++i) {
            const int u = ub + i;
            if (u >= units) break;
            const int g = u / ntile, t = u - g * ntile;
            const int span = min(64 * t + 64, n) - 64 * t;
            uint32_t acc_l = 0, acc_n = 0;
            // halves kept by hm: a half is not -inf when (w & hm) ^ (hm & -inf)
            // is not zero there, not +-0 when w & hm & 0x7FFF is not
            auto scan_chunk = [&](int bt, const uint32_t (&hm)[4]) {
                uint32_t tl = 0, tn = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    tl |= (w[i][bt][j] & hm[j]) ^ (hm[j] & 0xFC00FC00u);
                    tn |= w[i][bt][j] & hm[j];
                }
                if (okr[i][bt]) {
                    acc_l |= tl;
                    acc_n |= tn & 0x7FFF7FFFu;
                }
            };
            if (t != ntile_all - 1) {
#pragma unroll
                for (int bt = 0; bt < 5; ++bt) scan_chunk(bt, hmi[bt]);
            } else {
                // the last tile ends at n
#pragma unroll
                for (int bt = 0; bt < 5; ++bt) {
                    const uint32_t m8 = m8i[bt] & entry_range(0, min(last_span - 8 * lc + mis2[bt], 8));
                    const uint32_t hm[4] = {half_mask(m8, 0), half_mask(m8, 1), half_mask(m8, 2), half_mask(m8, 3)};
                    scan_chunk(bt, hm);
                }
            }
            const bool live = __any(acc_l != 0);
            const bool nonzero = __any(acc_n != 0);
            uint32_t bits = (live ? 1u : 0u) | (nonzero ? 2u : 0u);
            if (live && span < 64) bits = 3u;
            if (live) { tlo = min(tlo, t); thi = max(thi, t); }
            if (lane == 0) flags[g * PF_MAXT + t] = (uint8_t)bits;
        }
    };
    if (wave * UB < units) batch(wave * UB, true);
    else after_loads();
    for (int ub = wave * UB + NWV * UB; ub < units; ub += NWV * UB) batch(ub, false);
    if (lane == 0) { red[2 * wave] = tlo; red[2 * wave + 1] = thi; }
    lds_barrier();
    tlo = red[0];
    thi = red[1];
#pragma unroll
    for (int wv = 1; wv < NWV; ++wv) { tlo = min(tlo, red[2 * wv]); thi = max(thi, red[2 * wv + 1]); }
    lds_barrier();   // red may be reused by the caller
    if (ntile_all > PF_MAXT) {   // unclassified tail: keep it in the range
        tlo = min(tlo, PF_MAXT);
        thi = ntile_all - 1;
    }
    if (thi < 0) { lo = 0; hi = 0; } else { lo = 64 * tlo; hi = min(64 * thi + 64, n); }
}

// MM: 0 no mask, 1 an F16 mask tensor, 2 an implicit causal / window mask
// (query row i attends kv j iff j <= i + offset and, with a window W,
// j >= i + offset - W + 1), which equals the tensor holding 0 there and -inf
// elsewhere; its live range and tile classes follow from the formula, and a
// mixed tile's mask words are formed in registers, bit for bit those the
// tensor would give.
template <int D, int NQW, int KVG, int MM, bool QF16>
__global__ __launch_bounds__(64 * NQW * KVG) void fa_prefill_kernel(AttnArgs a, GridMap gm) {
    static_assert(D == 64 || D == 128, "head dim");
    constexpr bool MASK = MM != 0;
    constexpr bool IMPL = MM == 2;
    constexpr int NW = NQW * KVG;      // wavefronts
    constexpr int NT = 64 * NW;
    constexpr int BM = 32 * NQW;
    constexpr int BS = PF_BN * KVG;    // KV positions per step
    constexpr int KS = D / 16;         // S-MFMA k-steps
    constexpr int DB = D / 32;         // O^T row blocks
    constexpr int CH = D / 8;          // 16-byte chunks per row
    constexpr int ROWS_PER_LOAD = 64 / CH;   // rows one wavefront instruction fills
    constexpr int NLOAD = BS * CH / NT;      // instructions per wavefront per matrix per step
    static_assert(NLOAD * NT == BS * CH, "step split");
    constexpr int TILE_BYTES = BS * D * 2;   // one matrix of one step
    constexpr int NE = 16 * DB;              // O elements per lane
    constexpr int XSLOT = NQW * 64;          // floats per published O element
    static_assert((KVG - 1) * NE * XSLOT * 4 <= 4 * TILE_BYTES, "merge buffers");

    // V first: its reads (twice as many as K's) then need no base register
    __shared__ __attribute__((aligned(16))) char sV[2 * TILE_BYTES];
    __shared__ __attribute__((aligned(16))) char sK[2 * TILE_BYTES];
    __shared__ float s_ml[KVG > 1 ? 2 * (KVG - 1) * NQW * 64 : 1];
    __shared__ int s_red[2 * NW];
    __shared__ uint8_t s_tflag[MM == 1 ? NQW * PF_MAXT : 1];

    // ---- XCD-aware position of this workgroup --------------------------------
    int qt, h, b, hk, bkv;
    gm.locate(blockIdx.x, qt, h, b, hk, bkv);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qw = wave % NQW;
    const int kg = wave / NQW;
    const int q0 = qt * BM;
    const char* kb = (const char*)a.k + (int64_t)hk * a.k_nb2 + (int64_t)bkv * a.k_nb3;
    const char* vb = (const char*)a.v + (int64_t)hk * a.v_nb2 + (int64_t)bkv * a.v_nb3;

    const int nl = lane & 31;
    const int hh = lane >> 5;
    const int qrow = q0 + qw * 32 + nl;
    const bool qvalid = qrow < a.nq;
    const int nstep = (a.nkv + BS - 1) / BS;         // BS-position steps

    // ---- Q operand (B of S^T = K Q^T): row qrow, dims 16ks + 8hh .. +7 ----
    // (the Q element type is a template parameter: a load-or-convert branch on
    // it makes the compiler wait for all global loads inside the KV loop).
    // Rows past n_q load row 0 and are zeroed. All loads issue back to back
    // (with a mask tensor, right after the mask scan's first loads); F32 rows
    // are held raw and rounded (and rotated) only after the first KV step's
    // loads are issued, so the first step's loads do not wait for Q. (A branch
    // on the rotation between one row chunk's loads and the next would make
    // the compiler wait for each chunk in turn.)
    half8 qb[KS];
    floatx4 qraw[QF16 ? 1 : KS][2];
    int qpos = 0;   // rotary position of row qrow
    auto issue_q = [&]() {
        const int64_t qoff = (int64_t)(qvalid ? qrow : 0) * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if constexpr (QF16) {
                qb[ks] = *(const half8*)((const char*)a.q + qoff + (int64_t)(16 * ks + 8 * hh) * 2);
            } else {
                const floatx4* p = (const floatx4*)((const char*)a.q + qoff + (int64_t)(16 * ks + 8 * hh) * 4);
                qraw[ks][0] = p[0];
                qraw[ks][1] = p[1];
            }
        }
        if constexpr (!QF16) {
            // issued with the Q loads and without a branch (one would make the
            // compiler wait for every load before it); without a rotary
            // embedding it reads the first word of Q, unused
            const int* pp = a.rope_pos ? a.rope_pos + ((int64_t)b * a.nq + (qvalid ? qrow : 0)) : (const int*)a.q;
            qpos = *pp;
        }
    };
    // With a mask tensor the scan's loads go first and Q's follow them at
    // once, so the scan waits for its own loads only.
    if constexpr (MM != 1) issue_q();
    // With a mask tensor, first one word of every 128-byte line of the step a
    // causal mask starts with (step 0) is read into registers, so that its
    // K/V are on their way to L2 while the scan runs and its LDS copies,
    // issued after the scan, find them there. These are plain loads the
    // compiler sees (their registers stay theirs until the words are consumed
    // below); the copies themselves are not issued before the scan.
    constexpr int WLPR = D / 64;                      // 128-byte lines per K/V row
    constexpr int WARM = (BS * WLPR + NT - 1) / NT;   // lines per thread per matrix
    uint32_t warm[MM == 1 ? 2 * WARM : 1];
    if constexpr (MM == 1) {
        const int wrows = min(BS, a.nkv);
#pragma unroll
        for (int u = 0; u < WARM; ++u) {
            const int line = min(tid + NT * u, wrows * WLPR - 1);
            const int64_t wr = line / WLPR;
            warm[2 * u] = *(const uint32_t*)(kb + wr * a.k_nb1 + (line % WLPR) * 128);
            warm[2 * u + 1] = *(const uint32_t*)(vb + wr * a.v_nb1 + (line % WLPR) * 128);
        }
    }
    // rounds the F32 rows to f16 (ggml's Q conversion), rotating them first
    // when a rotary embedding is given; zeroes rows past n_q
    // (The rotation's angles come from one running product over the row's
    // pairs, as ggml builds its cos / sin cache: pair 8 ks + o, o < 8, belongs
    // to the lanes with hh = o / 4, which keep it for their slot o % 4; a
    // product loop restarted for every ks cost ~6 instructions per step.)
    auto finish_q = [&]() {
        if constexpr (!QF16) {
            float th = (float)qpos;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                float x[8] = {qraw[ks][0][0], qraw[ks][0][1], qraw[ks][0][2], qraw[ks][0][3],
                              qraw[ks][1][0], qraw[ks][1][1], qraw[ks][1][2], qraw[ks][1][3]};
                if (a.rope_pos) {
                    float ang[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int o = 0; o < 8; ++o) {
                        if (ks > 0 || o > 0) th *= a.rope_ts;
                        if ((o >> 2) == hh) ang[o & 3] = th;
                    }
                    rope8_ang(x, ang, 16 * ks + 8 * hh, a.rope_dims);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) qb[ks][e] = (_Float16)x[e];
            }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            if (!qvalid) qb[ks] = half8{0, 0, 0, 0, 0, 0, 0, 0};
    };

    // ---- live column range and tile classes of the mask over this workgroup's
    // rows ----------------------------------------------------------------------
    // Steps wholly outside the range are never loaded. Inside it, a wavefront's
    // tile whose entries are all -inf is skipped, one whose entries are all
    // zero is computed without reading the mask, and only mixed tiles (the
    // diagonal of a causal mask, the edges of a window) read mask values.
    const uint16_t* mplane = nullptr;
    int step_lo = 0, step_hi = nstep;
    if constexpr (MM == 1) {
        mplane = (const uint16_t*)((const char*)a.mask + (int64_t)(h % a.hm) * a.m_nb2 +
                                   (int64_t)(b % a.bm) * a.m_nb3);
        int lo = 0, hi = 0;
        const int rows = min(BM, a.nq - q0);
        mask_scan_tiles<NT, NQW>((const uint16_t*)((const char*)mplane + (int64_t)q0 * a.m_nb1), a.m_nb1, rows,
                                 a.nkv, s_tflag, s_red, lo, hi, issue_q);
        step_lo = lo / BS;
        step_hi = hi > lo ? (hi - 1) / BS + 1 : 0;
    } else if constexpr (IMPL) {
        // rows q0 .. q_last attend [q0 + offset - W + 1, q_last + offset]
        const int64_t q_last = (int64_t)min(q0 + BM, a.nq) - 1;
        int64_t lo = a.im_window > 0 ? (int64_t)q0 + a.im_offset - a.im_window + 1 : 0;
        int64_t hi = q_last + a.im_offset + 1;
        lo = lo < 0 ? 0 : lo;
        hi = hi > a.nkv ? a.nkv : hi;
        if (hi > lo) {
            step_lo = (int)(lo / BS);
            step_hi = (int)((hi - 1) / BS) + 1;
        } else {
            step_lo = step_hi = 0;
        }
    }
    // Step sequence. Without a mask: every step, the last one (which holds
    // the partial tile when n_kv % 64 != 0) last, the others rotated by the
    // query block. With a mask: the steps of the live range, in order.
    // -1 ends the sequence.
    int n_left = nstep - 1;   // steps after the current one (sequence of all steps)
    auto next_step = [&](int s) -> int {
        if (!MASK) {
            if (n_left <= 0) return -1;
            if (--n_left == 0) return nstep - 1;
            return s + 2 == nstep ? 0 : s + 1;
        }
        return s + 1 < step_hi ? s + 1 : -1;
    };
    int first = -1;
    if (!MASK) first = nstep == 1 ? 0 : (int)(((int64_t)qt * (nstep - 1)) / (int)gm.nqt);
    else if (step_lo < step_hi) first = step_lo;

    // ---- step loads: global -> LDS ------------------------------------------
    // Instruction i of wavefront w fills rows [ROWS_PER_LOAD * (w + NW i), + ROWS_PER_LOAD)
    // of the step; lane l writes LDS chunk l % CH of row + l / CH, which holds
    // the row's chunk (l % CH) ^ swizzle(row). A step's rows start at a scalar
    // base; each lane adds a 32-bit offset fixed for the whole walk (row
    // strides are below 8 MiB, checked by the host). The last step clamps
    // rows past n_kv to row n_kv - 1 instead.
    const int ld_row = lane / CH;
    uint32_t ldk[NLOAD], ldv[NLOAD];
    int colk[NLOAD], colv[NLOAD];
#pragma unroll
    for (int i = 0; i < NLOAD; ++i) {
        const int r = ROWS_PER_LOAD * (wave + NW * i) + ld_row;
        colk[i] = ((lane % CH) ^ swz_k<D>(r)) * 16;
        colv[i] = ((lane % CH) ^ swz_v<D>(r)) * 16;
        ldk[i] = (uint32_t)r * (uint32_t)a.k_nb1 + colk[i];
        ldv[i] = (uint32_t)r * (uint32_t)a.v_nb1 + colv[i];
    }
    const uint32_t lds_k = lds_offset(sK), lds_v = lds_offset(sV);
    auto issue_step = [&](int s, int stg) {
        const int kv0 = __builtin_amdgcn_readfirstlane(s) * BS;   // s is uniform
        const uint32_t k_dst = lds_k + stg * TILE_BYTES, v_dst = lds_v + stg * TILE_BYTES;
        if (kv0 + BS <= a.nkv) {
            const char* kst = kb + (int64_t)kv0 * a.k_nb1;
            const char* vst = vb + (int64_t)kv0 * a.v_nb1;
#pragma unroll
            for (int i = 0; i < NLOAD; ++i) {
                const uint32_t r0b = ROWS_PER_LOAD * (wave + NW * i) * D * 2;
                dma16(kst, ldk[i], k_dst + r0b);
                dma16(vst, ldv[i], v_dst + r0b);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NLOAD; ++i) {
                const int r0 = ROWS_PER_LOAD * (wave + NW * i);
                const int kv = min(kv0 + r0 + ld_row, a.nkv - 1);
                dma16_addr(kb + (int64_t)kv * a.k_nb1 + colk[i], k_dst + r0 * D * 2);
                dma16_addr(vb + (int64_t)kv * a.v_nb1 + colv[i], v_dst + r0 * D * 2);
            }
        }
    };

    floatx16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    // K row this lane fetches as A-operand row nl of each 32-block, within this
    // wavefront's 64-position tile of the step; kaddr[ks] = byte offset of its
    // chunk 2 ks + hh (32-block kvb adds 32 rows, stage adds TILE_BYTES)
    int kaddr[KS];
    {
        const int am = nl >> 3, ahb = (nl >> 2) & 1, ab = nl & 3;
        const int krow = PF_BN * kg + (ahb ? 16 + ((am + 2) & 3) * 4 + ab : 4 * am + ab);
        const int kx = hh ^ swz_k<D>(krow);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kaddr[ks] = krow * D * 2 + ((2 * ks) ^ kx) * 16;
    }
    // V^T reads of operand pc = 2 kvb + cc: lane reads row kvl + 4 hi + vq of
    // the tile, vq = (lane % 16) / 4, kvl = 32 kvb + (hh ? 24 - 8 cc : 8 cc) (the
    // 8 positions of P operand pc), and the 8 bytes at dims 32 db + 16 ((lane %
    // 32) / 16) + 4 (lane % 4), i.e. chunk 4 db + clo, clo = 2 ((lane % 32) / 16)
    // + (lane % 4) / 2. vaddr[cc][db] = byte offset for kvb = 0, hi = 0.
    int vaddr[2][DB];
    {
        const int vq = (lane & 15) >> 2;
        const int clo = 2 * ((lane & 31) >> 4) + ((lane & 3) >> 1);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int db = 0; db < DB; ++db)
                vaddr[cc][db] = (PF_BN * kg + (hh ? 24 - 8 * cc : 8 * cc) + vq) * D * 2 +
                                ((4 * db + clo) ^ swz_v<D>(vq)) * 16 + (lane & 1) * 8;
    }
    // mask row of this lane's query (rows past n_q read row 0: their results
    // are never stored)
    const uint16_t* mrow = nullptr;
    if (MM == 1) mrow = (const uint16_t*)((const char*)mplane + (int64_t)(qvalid ? qrow : 0) * a.m_nb1);
    const half2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    const float c = a.scale_log2;

    // Mask of the tile at kv0, as f16 pairs: element j of score block kvb is
    // half (j % 2) of mw[kvb][j / 2]. Lane half 0 holds positions 32 kvb +
    // 0..15 in order; lane half 1 holds 32 kvb + 16 + ((j + 8) % 16), the
    // row-to-KV mapping, so its two 16-byte loads come swapped. Positions
    // past n_kv read as -inf.
    auto load_mask = [&](int kv0, uint32_t (&mw)[2][8]) {
        if constexpr (IMPL) {
            // implicit: 0 where the row attends kv, -inf elsewhere (and past
            // n_kv); rows past n_q use row 0, as the tensor path reads
            const int64_t last = (int64_t)(qvalid ? qrow : 0) + a.im_offset;
            const int64_t first = a.im_window > 0 ? last - a.im_window + 1 : INT64_MIN;
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    uint32_t pair = 0;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int kv = kv0 + 32 * kvb + pf_kv_of(hh, 2 * w + e);
                        const bool live = kv < a.nkv && (int64_t)kv <= last && (int64_t)kv >= first;
                        pair |= (live ? 0u : (uint32_t)kF16NegInf) << (16 * e);
                    }
                    mw[kvb][w] = pair;
                }
        } else if (a.mask_vec && kv0 + PF_BN <= a.nkv) {
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb) {
                const uint16_t* p = mrow + kv0 + 32 * kvb + 16 * hh;
                const u32x4 lo = *(const u32x4*)(p + 8 * hh);
                const u32x4 hi = *(const u32x4*)(p + 8 - 8 * hh);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    mw[kvb][w] = lo[w];
                    mw[kvb][4 + w] = hi[w];
                }
            }
        } else {
            // element loads from a clamped position, positions past n_kv
            // replaced afterwards: a load under a branch makes the compiler
            // wait for it before issuing the next one
            uint16_t raw[2][16];
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int j = 0; j < 16; ++j) raw[kvb][j] = mrow[min(kv0 + 32 * kvb + pf_kv_of(hh, j), a.nkv - 1)];
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    uint32_t pair = 0;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int kv = kv0 + 32 * kvb + pf_kv_of(hh, 2 * w + e);
                        const uint32_t bits = kv < a.nkv ? (uint32_t)raw[kvb][2 * w + e] : kF16NegInf;
                        pair |= bits << (16 * e);
                    }
                    mw[kvb][w] = pair;
                }
        }
    };

    // One 64-position tile at kv0 from LDS stage stg.
    // TAIL: the tile runs past n_kv (positions >= n_kv are forced to -inf).
    // M: add the mask words mw (a mixed tile); without M the tile is computed
    // as unmasked (no mask, or a tile whose mask entries are all zero, which
    // never runs past n_kv: entries there read as -inf).
    auto tile = [&](auto tail_tag, auto mask_tag, int stg, int kv0, const uint32_t (&mw)[2][8]) {
        constexpr bool M = decltype(mask_tag)::value;
        constexpr bool TAIL = !M && decltype(tail_tag)::value;   // the mask path covers the tail
        if constexpr (M) {
            bool any = false;
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int w = 0; w < 8; ++w) any |= mw[kvb][w] != 0xFC00FC00u;
            if (!__any(any)) return;
        }
        const char* ks_ = sK + stg * TILE_BYTES;
        const char* vs_ = sV + stg * TILE_BYTES;

        floatx16 S[2];
#pragma unroll
        for (int kvb = 0; kvb < 2; ++kvb) {
#pragma unroll
            for (int j = 0; j < 16; ++j) S[kvb][j] = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 ka = *(const half8*)(ks_ + kaddr[ks] + 32 * kvb * D * 2);
                S[kvb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb[ks], S[kvb], 0, 0, 0);
            }
        }

        // Row max in log2 units. Without a mask the scale is applied after the
        // max (max(c*s) = c*max(s) for c >= 0, c*min(s) for c < 0) and folded
        // into the exp2 argument, one FMA per score.
        float mx;
        if (M || TAIL) {
            mx = -INFINITY;
#pragma unroll
            for (int kvb = 0; kvb < 2; ++kvb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    float x = S[kvb][j] * c;
                    if constexpr (M) {
                        const half2 m2 = __builtin_bit_cast(half2, mw[kvb][j >> 1]);
                        x = fmaf((float)m2[j & 1], kLog2e, x);   // -inf stays -inf
                    }
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
                const float e = (M || TAIL) ? S[kvb][8 * cc + i] - msafe : fmaf(S[kvb][8 * cc + i], c, -msafe);
                pb[i] = (_Float16)exp2_fast(e);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                half2 p2 = {pb[2 * i], pb[2 * i + 1]};
                lsum[i & 1] = __builtin_amdgcn_fdot2(p2, ones, lsum[i & 1], false);
            }
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const char* p = vs_ + vaddr[cc][db] + 32 * kvb * D * 2;
                const half4 lo4 = lds_read_tr16(p);
                const half4 hi4 = lds_read_tr16(p + 4 * D * 2);
                const half8 va = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[db], 0, 0, 0);
            }
        }
        l_run += lsum[0] + lsum[1];
    };

    // One step: start loading step s_nxt into stage STG ^ 1 (and, under a
    // mask, the mask words of its tile), compute step s_cur from stage STG
    // (full tiles, or any tile under a mask), then wait for the loads and for
    // every wavefront. The stage is a template constant so every LDS read
    // address is a register plus an immediate.
    uint32_t mwa[2][8], mwb[2][8];
    // class of this wavefront's tile at kv0 (MASK only): 1 all zero, 2 or 0
    // dead, 3 mixed
    auto tclass = [&](int kv0) -> int {
        if constexpr (IMPL) {
            const int64_t r0 = q0 + 32 * qw;                           // this wavefront's rows
            const int64_t r1 = (int64_t)min(q0 + 32 * qw + 32, a.nq) - 1;
            if (r1 < r0) return 0;
            const int64_t c0 = kv0, c1 = (int64_t)min(kv0 + PF_BN, a.nkv) - 1;   // the tile's columns
            const int64_t off = a.im_offset, W = a.im_window;
            if (c0 > r1 + off || (W > 0 && c1 < r0 + off - W + 1)) return 2;
            const bool all = c1 <= r0 + off && (W == 0 || c0 >= r1 + off - W + 1);
            return (all && kv0 + PF_BN <= a.nkv) ? 1 : 3;
        } else {
            const int t = kv0 / PF_BN;
            return t < PF_MAXT ? (int)s_tflag[qw * PF_MAXT + t] : 3;
        }
    };
    auto run_tile = [&](int stg, int kv0, const uint32_t (&mw)[2][8]) {
        if constexpr (MASK) {
            const int f = tclass(kv0);
            if (f == 3) tile(std::false_type{}, std::true_type{}, stg, kv0, mw);
            else if (f == 1) tile(std::false_type{}, std::false_type{}, stg, kv0, mw);
        } else {
            tile(std::false_type{}, std::false_type{}, stg, kv0, mw);
        }
    };
    auto run_step = [&](auto stg_tag, int s_cur, int s_nxt, const uint32_t (&mw_cur)[2][8], uint32_t (&mw_nxt)[2][8]) {
        constexpr int STG = decltype(stg_tag)::value;
        if (s_nxt >= 0) {
            issue_step(s_nxt, STG ^ 1);
            const int kv0n = s_nxt * BS + PF_BN * kg;
            if (MASK && kv0n < a.nkv && tclass(kv0n) == 3) load_mask(kv0n, mw_nxt);
        }
        const int kv0 = s_cur * BS + PF_BN * kg;
        if (kv0 < a.nkv) run_tile(STG, kv0, mw_cur);
        wait_all_mem();
        __syncthreads();
    };

    // Stage 0 and stage 1 alternate. Without a mask the last step of the
    // sequence (it may hold the partial tile) is left for after the loop.
    int s_cur = first;
    int last_stage = 0;
    if (s_cur >= 0) {
        issue_step(s_cur, 0);
        const int kv0 = s_cur * BS + PF_BN * kg;
        if (MASK && kv0 < a.nkv && tclass(kv0) == 3) load_mask(kv0, mwa);
    }
    finish_q();
    if constexpr (MM == 1) {   // the words warming step 0 (their wait joins the one below)
        uint32_t wsum = 0;
#pragma unroll
        for (int u = 0; u < 2 * WARM; ++u) wsum ^= warm[u];
        asm volatile("" ::"v"(wsum));
    }
    wait_all_mem();
    __syncthreads();
    while (s_cur >= 0) {
        int s_nxt = next_step(s_cur);
        if (!MASK && s_nxt < 0) { last_stage = 0; break; }
        run_step(std::integral_constant<int, 0>{}, s_cur, s_nxt, mwa, mwb);
        s_cur = s_nxt;
        if (s_cur < 0) break;
        s_nxt = next_step(s_cur);
        if (!MASK && s_nxt < 0) { last_stage = 1; break; }
        run_step(std::integral_constant<int, 1>{}, s_cur, s_nxt, mwb, mwa);
        s_cur = s_nxt;
    }
    if (!MASK && s_cur >= 0) {
        const int kv0 = s_cur * BS + PF_BN * kg;
        if (kv0 < a.nkv) tile(std::true_type{}, std::false_type{}, last_stage, kv0, mwa);   // mask words unused
        __syncthreads();
    }

    // ---- merge the KV groups (LDS), normalise, store dst[b][qrow][h][d] ------
    if constexpr (KVG > 1) {
        // groups 1.. publish (m, l, O) element-major, so a wavefront's 64
        // lanes write consecutive words; the stage arrays are free after the
        // last barrier. Element e of group g goes to slot (g - 1) * NE + e of
        // XSLOT floats, filling sV and then sK.
        constexpr int SLOTS_V = 2 * TILE_BYTES / (XSLOT * 4);
        const int slot = qw * 64 + lane;
        auto xo_at = [&](int g, int e) -> float* {
            const int L = (g - 1) * NE + e;
            return L < SLOTS_V ? (float*)sV + L * XSLOT + slot : (float*)sK + (L - SLOTS_V) * XSLOT + slot;
        };
        float* xm = s_ml;
        float* xl = s_ml + (KVG - 1) * NQW * 64;
        if (kg > 0) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 16; ++j) *xo_at(kg, db * 16 + j) = o[db][j];
            xm[(kg - 1) * NQW * 64 + slot] = m_run;
            xl[(kg - 1) * NQW * 64 + slot] = l_run;
        }
        __syncthreads();
        if (kg > 0) return;
        float M = m_run;
#pragma unroll
        for (int g = 1; g < KVG; ++g) M = fmaxf(M, xm[(g - 1) * NQW * 64 + slot]);
        const float Ms = (M == -INFINITY) ? 0.f : M;
        const float w0 = exp2_fast(m_run - Ms);
        l_run *= w0;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[db][j] *= w0;
#pragma unroll
        for (int g = 1; g < KVG; ++g) {
            const float wg = exp2_fast(xm[(g - 1) * NQW * 64 + slot] - Ms);
            l_run = fmaf(wg, xl[(g - 1) * NQW * 64 + slot], l_run);
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 16; ++j) o[db][j] = fmaf(wg, *xo_at(g, db * 16 + j), o[db][j]);
        }
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

template <int D, int NQW, int KVG, int MM>
static hipError_t launch_pw(const AttnArgs& a, hipStream_t st) {
    constexpr int BM = 32 * NQW;
    const int nqt = (a.nq + BM - 1) / BM;
    const int64_t nwg = (int64_t)nqt * a.hq * a.b;
    if (nwg <= 0 || nwg > 0x7fffffff) return hipErrorInvalidValue;
    constexpr int NT = 64 * NQW * KVG;
    // under a mask, heavy query tiles first (a causal or window mask makes
    // later tiles walk more steps)
    const GridMap gm = MM != 0 ? GridMap::make_tiles_desc((int)nwg, nqt, a.hq, a.hkv, a.b, a.bk)
                               : GridMap::make((int)nwg, nqt, a.hq, a.hkv, a.b, a.bk);
    const dim3 grid((unsigned)nwg), block(NT);
    if (a.q_f16) hipLaunchKernelGGL((fa_prefill_kernel<D, NQW, KVG, MM, true>), grid, block, 0, st, a, gm);
    else hipLaunchKernelGGL((fa_prefill_kernel<D, NQW, KVG, MM, false>), grid, block, 0, st, a, gm);
    return hipGetLastError();
}

// waves = query-row wavefronts per workgroup (32 rows each); 0 picks the
// default. hd 64 without a mask: 4 (16 wavefronts with their 3 KV partners,
// 4 per SIMD) or 2. hd 64 with a mask keeps its mask words in registers and
// always runs 2 (8 wavefronts). hd 128: 4 or 2 with one KV partner each; with
// a mask (tensor or implicit) always 2.
hipError_t launch_prefill(const AttnArgs& a, int head_dim, int waves, hipStream_t st) {
    const int mm = a.im_causal ? 2 : (a.mask != nullptr ? 1 : 0);
    if (head_dim == 64) {
        if (mm == 1) return launch_pw<64, 2, 4, 1>(a, st);
        if (mm == 2) return launch_pw<64, 2, 4, 2>(a, st);
        if (waves == 0 || waves == 4) return launch_pw<64, 4, 4, 0>(a, st);
        if (waves == 2) return launch_pw<64, 2, 4, 0>(a, st);
    } else if (head_dim == 128) {
        // masked hd 128 always runs 2 (with 4 its registers spill)
        if (mm == 1) return launch_pw<128, 2, 2, 1>(a, st);
        if (mm == 2) return launch_pw<128, 2, 2, 2>(a, st);
        if (waves == 0 || waves == 4) return launch_pw<128, 4, 2, 0>(a, st);
        if (waves == 2) return launch_pw<128, 2, 2, 0>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace vxfa
