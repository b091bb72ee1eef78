// fa_decode.hip — single-query (decode-step) attention against a KV cache,
// split over the KV length, for gfx950. One launch per call.
//
// Replaces the backend kernel of GGML_OP_FLASH_ATTN_EXT for the decode calls
// voxtral.cpp makes from build_decoder_layer (src/voxtral.cpp:1802) with
// n_tokens = 1 (step graphs :1959-1962 and :2050-2053), where every KV head
// serves G = Hq / Hkv query heads (32 / 8 = 4). The cache is f16 (the
// configured layout) or F32 (the reference's own cache type,
// src/voxtral.cpp:1126-1136); against F32 K/V both products are F32, as in
// ggml's CPU kernel for F32 K (Q is not rounded to f16).
//
// Two kernels on the caller's stream:
//   fa_decode         grid (n_split * Hkv, B), kDecodeWaves wavefronts per
//                     workgroup, the kv head fastest-varying (neighbouring
//                     workgroups stream neighbouring head slices of the same
//                     cache rows). Each workgroup reduces one contiguous slice
//                     of the live KV range to (O, m, l) per query head of its
//                     group; with n_split == 1 it writes the output directly.
//   fa_decode_combine grid (Hq * D / 32, B), one wavefront per (query head,
//                     32 output dims): log-sum-exp merge of the n_split
//                     partials in a fixed order (deterministic output); runs
//                     only when n_split > 1. Its workgroups take the kv head
//                     fastest, as the split kernel's do, so (with 8 kv heads)
//                     the merge of kv head g runs on the XCD whose workgroups
//                     wrote g's records and reads them from that XCD's L2
//                     (workgroups go to the 8 XCDs round robin).
// The kernel boundary orders the partial records' stores before the merge's
// loads. A merge inside the first kernel by the last workgroup of each
// (batch, kv head) to finish — records written with device-scope stores, a
// device-scope arrival counter, records read back with device-scope loads,
// no cache maintenance — was built and measured slower at n_kv 8192 (split
// work alone 11.4 us; waiting for the stores plus the counter +2.1 us; the
// last workgroup's merge +3.9 us, one CU pulling every record through
// device-scope round trips) than the kernel boundary plus a 128-workgroup
// combine (about 3 us); with device-scope fences instead it was +13 us (each
// fence writes back and invalidates the whole L2 of its XCD).
//
// Inside a wavefront (tiles of TP positions, 32 for f16 and 16 for F32 K/V,
// so a tile is 16 KB either way, and 16 for f16 on short spans, where tiles
// of 32 would leave the grid short of workgroups; software pipelined: the
// next tile's K/V loads are in flight while the current tile is computed):
//   QK^T  v_mfma_f32_16x16x32_f16 per (16 positions, 32 dims); against F32
//         K, v_mfma_f32_16x16x4f32 per (16 positions, 4 dims) with F32 Q.
//         The A operand holds the G query heads replicated 16/G times, so
//         every lane gets the scores of all G heads for one position: no
//         cross-lane dot reduction.
//   K     read like V, D / 8 lanes per row and 16 contiguous bytes per
//         lane, so one load instruction reads whole 256-byte head rows, then
//         turned through a wavefront-private LDS tile (rows in, 16-byte chunks
//         XOR-swizzled by row so the operand reads hit 16 bank groups) into
//         the MFMA B-operand layout. Against K read straight in that layout
//         (16 positions x 64 contiguous bytes per load instruction), A/B on
//         one box, us per layer: n_kv 1024 7.47 -> 7.11, 8192 11.37 -> 10.94,
//         rope + append 14.05 -> 12.7, F32 cache 20.1 -> 19.3, sliding window
//         with an implicit mask 7.97 -> 7.42, 32 ragged streams 135 -> 133.5
//         (a streaming probe of the two patterns alone: 8.0 -> 7.1 us at
//         n_kv 8192).
//   V     16 (hd128) or 8 (hd64) lanes per row, fully coalesced 128-bit
//         loads; P.V on the VALU with fp32 accumulators (each lane owns 8
//         dims of all G heads); P is handed from the MFMA layout to the V
//         layout through a 512-byte LDS slot per wavefront.
//   Softmax fp32, exp2 with scale*log2(e) folded in, one running max per head
//         shared by the wavefront (DPP row reductions).
// Masks: an additive F16 mask is honoured exactly (-inf removes a position).
// The workgroup first scans the mask row(s) for the live range, so a sliding
// window or a ragged stream length only costs its live positions. Without a
// mask tensor the host passes the live range (all of n_kv, or the rows an
// implicit causal / window mask leaves to the query) and sizes the splits to
// it, so no scan runs.
#include "fa_common.h"

#include <type_traits>

namespace vxfa {

constexpr int DEC_WAVES = kDecodeWaves;
constexpr int DEC_THREADS = 64 * DEC_WAVES;

// Log-sum-exp merge of the n_split partial records, one wavefront per
// (query head, 32 output dims):
//   M = max_s m_s,  w_s = 2^(m_s - M),  O = sum_s w_s O_s / sum_s w_s l_s.
// Lane (f, grp) = (lane % 8, lane / 8) takes splits grp, grp + 8, ... (MAXS
// of them, at least n_split / 8): float4 f of each one's slice and its
// (m, l). All loads issue back to back (loads past the last split read the
// last record again; their weights are zero), so the merge costs one memory
// round trip. The lane forms its splits' max, weights and sums itself; the
// eight split groups then combine over lanes l ^ 8, l ^ 16, l ^ 32 (a DPP
// row rotation and two lane-swap instructions, on the VALU: the former
// 64-lane LDS shuffles made three dependent chains of up to six round
// trips). Fixed order: the output is deterministic.
template <int D, int G, int MAXS>
__global__ __launch_bounds__(64) void fa_decode_combine(AttnArgs a) {
    constexpr int CSUB = D / 32;                  // 32-dim slices per head
    constexpr int CF4 = 8;                        // float4 per slice
    constexpr int NGRP = 64 / CF4;                // split groups
    constexpr int RS = dec_record_floats(D, G);
    static_assert(MAXS * NGRP <= kDecodeMaxSplit, "splits per lane");
    const int lane = threadIdx.x;
    // kv head fastest: with 8 kv heads the workgroups of kv head g run on XCD
    // g, where the split workgroups that wrote g's records ran, and read them
    // from its L2 (the kernel boundary writes them back but leaves them
    // valid there). Head-major, the records came from the other XCDs:
    // n_kv 8192 10.97 -> 10.48 us per layer, 1024 6.57 -> 6.18, a 2048
    // window with an implicit mask 7.14 -> 6.64 (alternating A/B on one box).
    const int g = (int)blockIdx.x % a.hkv, rest = (int)blockIdx.x / a.hkv;
    const int h = rest / CSUB, sl = rest % CSUB;
    const int hq = g * G + h;
    const int b = blockIdx.y;
    const int ns = a.n_split;
    const float* base = a.ws + (int64_t)(b * a.hkv + g) * ns * RS;
    const int f = lane % CF4, grp = lane / CF4;

    floatx4 o[MAXS];
    float mi[MAXS], li[MAXS];
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
        const float* rec = base + (int64_t)min(grp + i * NGRP, ns - 1) * RS;
        o[i] = *(const floatx4*)(rec + h * D + 32 * sl + 4 * f);
        mi[i] = rec[G * D + h];
        li[i] = rec[G * D + G + h];
    }
    // over the lanes l ^ 8, l ^ 16, l ^ 32 (the other split groups)
    auto grp_max = [](float x) {
        x = fmaxf(x, row_ror<8>(x));
        const int xi = __builtin_bit_cast(int, x);
        const auto r = __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
        x = fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
        return pair32_max(x);
    };
    auto grp_sum = [](float x) {
        x += row_ror<8>(x);
        const int xi = __builtin_bit_cast(int, x);
        const auto r = __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
        x = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
        return pair32_sum(x);
    };
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
        const bool live = grp + i * NGRP < ns;
        mi[i] = live ? mi[i] : -INFINITY;
        li[i] = live ? li[i] : 0.f;
        M = fmaxf(M, mi[i]);
    }
    M = grp_max(M);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float L = 0.f;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
        const float w = exp2_fast(mi[i] - Ms);   // 0 for an empty or absent split (m = -inf)
        L = fmaf(w, li[i], L);
        acc[0] = fmaf(w, o[i][0], acc[0]);
        acc[1] = fmaf(w, o[i][1], acc[1]);
        acc[2] = fmaf(w, o[i][2], acc[2]);
        acc[3] = fmaf(w, o[i][3], acc[3]);
    }
    L = grp_sum(L);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = grp_sum(acc[c]);
    if (grp == 0) {
        const float inv = (L == 0.f) ? 0.f : 1.0f / L;
        const floatx4 out = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        *(floatx4*)(a.dst + ((int64_t)b * a.hq + hq) * D + 32 * sl + 4 * f) = out;
    }
}

// the divisors of one decode launch: kv heads, splits, q batches per kv
// batch, mask head planes, mask batches
struct DecodeDivs {
    DivMod hkv, split, bgrp, hm, bm;
};

// two wavefronts per SIMD (256 registers per lane, arch + accumulation): the
// masked f16 variant otherwise took 256 + 2 and ran one per SIMD
template <int D, int G, bool QF16, bool MASK, bool KV32, bool RING, bool T16>
__global__ __launch_bounds__(DEC_THREADS, 2) void fa_decode(AttnArgs a, DecodeDivs dv) {
    static_assert(D == 64 || D == 128, "head dim");
    static_assert(G == 1 || G == 2 || G == 4, "GQA group");
    constexpr int KS = D / 32;        // MFMA k-steps of 32 dims
    // positions per tile: 32 for f16 K/V (16 KB of K and V), 16 for F32 (16 KB)
    // and for f16 on short spans (T16: twice the workgroups for the same span)
    constexpr int TP = (KV32 || T16) ? 16 : 32;
    static_assert(!(KV32 && T16), "F32 tiles are 16 positions already");
    constexpr int NG = TP / 16;       // 16-position MFMA groups per tile
    constexpr int CH = D / 8;         // lanes per V row (8 dims each)
    constexpr int RPI = 64 / CH;      // V rows covered by one load instruction
    constexpr int NV = TP / RPI;
    constexpr int ESZ = KV32 ? 4 : 2; // K/V element size
    constexpr int NCH = D / 8;        // 16-byte chunks of an f16 row

    __shared__ floatx4 lds_p[DEC_WAVES][TP];
    __shared__ float lds_acc[DEC_WAVES][G][D];
    __shared__ float lds_m[DEC_WAVES][G];
    __shared__ float lds_l[DEC_WAVES][G];
    __shared__ int lds_red[2 * DEC_WAVES];
    // the group's query heads [G][D]: f16 against f16 K, F32 against F32 K
    __shared__ __align__(16) char lds_q_raw[G * D * (KV32 ? 4 : 2)];
    __shared__ float2 lds_rope[D / 2];   // cos / sin of each pair's rotary angle (with rope_pos)
    // each wavefront's K tile: TP rows of f16 (f16 K) or F32 (F32 K), 8 KiB either way
    __shared__ __align__(16) char lds_kt_raw[DEC_WAVES * TP * D * ESZ];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform (a scalar register): tile indices, row bases and loop
    // bounds derived from it stay on the scalar unit
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = (int)dv.hkv.mod(blockIdx.x);
    const int split = (int)dv.hkv.div(blockIdx.x);
    const int b = blockIdx.y;
    const int bkv = (int)dv.bgrp.div(b);
    constexpr bool masked = MASK;  // compile time, like QF16, so no load is conditional at run time
    // rotary position of the query token (also the appended row's: the host
    // requires one kv batch per q batch), requested before any other load. A
    // vector load (the opaque zero offset keeps it off the scalar unit, whose
    // out-of-order returns would make the first wait for kernel arguments
    // wait for it too); the in-order vector count then waits for it alone.
    // The load is unconditional (without rotary positions it reads a word of
    // the K cache and ignores it): a branch around it would keep the wait
    // for it next to it.
    int rope_p;
    {
        const int32_t* rp = a.rope_pos ? a.rope_pos + b : reinterpret_cast<const int32_t*>(a.k);
        int z;
        asm volatile("v_mov_b32 %0, 0" : "=v"(z));
        rope_p = rp[z];
    }

    // ---- live range of the KV axis -------------------------------------
    // The mask rows of this group's query heads: planes (g G + j) % hm of
    // batch b % bm. One scan when they are one plane or consecutive planes.
    int lo = a.kv_lo, hi = a.kv_hi;   // without a mask tensor the host gives the live range
    if constexpr (masked) {
        const char* mb = (const char*)a.mask + (int64_t)dv.bm.mod(b) * a.m_nb3;
        const int p0 = (int)dv.hm.mod(g * G);
        const int np = a.hm == 1 ? 1 : (p0 + G <= a.hm ? G : 0);
        if (np > 0) {
            mask_live_range<DEC_THREADS>((const uint16_t*)(mb + (int64_t)p0 * a.m_nb2), a.m_nb2, np, a.nkv, lds_red,
                                         lo, hi);
        } else {
            lo = 0x7fffffff;
            hi = 0;
            for (int j = 0; j < G; ++j) {
                int l1, h1;
                mask_live_range<DEC_THREADS>((const uint16_t*)(mb + (int64_t)dv.hm.mod(g * G + j) * a.m_nb2), 0, 1,
                                             a.nkv, lds_red, l1, h1);
                if (h1 > l1) { lo = min(lo, l1); hi = max(hi, h1); }
            }
            if (hi == 0) lo = 0;
        }
    }

    // With a fused append the new row (n_kv - 1) is not read from the cache:
    // every workgroup walks [lo, hi_main) and wavefront 0 of the last split
    // folds the new row in afterwards, from the F32 source.
    const bool new_live = a.append && hi == a.nkv;
    const int hi_main = a.append ? min(hi, a.nkv - 1) : hi;
    const int span = max(hi_main - lo, 0);
    const int ntiles = (span + TP - 1) / TP;
    // (ntiles * n_split < 2^31 but for caches of more than 2^30 positions)
    int t_begin, t_end;
    if (ntiles < (1 << 25)) {
        t_begin = (int)dv.split.div((uint32_t)(ntiles * split));
        t_end = (int)dv.split.div((uint32_t)(ntiles * (split + 1)));
    } else {
        t_begin = (int)(((int64_t)ntiles * split) / a.n_split);
        t_end = (int)(((int64_t)ntiles * (split + 1)) / a.n_split);
    }

    const char* kb = (const char*)a.k + (int64_t)g * a.k_nb2 + (int64_t)bkv * a.k_nb3;
    const char* vb = (const char*)a.v + (int64_t)g * a.v_nb2 + (int64_t)bkv * a.v_nb3;
    const uint16_t* mplane[4] = {nullptr, nullptr, nullptr, nullptr};
    if constexpr (masked) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hq = g * G + (i % G);
            mplane[i] = (const uint16_t*)((const char*)a.mask + (int64_t)dv.hm.mod(hq) * a.m_nb2 +
                                          (int64_t)dv.bm.mod(b) * a.m_nb3);
        }
    }

    const int vrow = lane / CH;           // row offset owned in the K / V load layout
    const int vcol = (lane % CH) * 8;     // dims owned in the K / V load layout

    // One tile in registers: K and V in the load layout (entry i = row
    // vrow + RPI i, dims vcol .. vcol + 7), mask entries of the lane's MFMA
    // position (16 grp + lane % 16) for its four accumulator rows.
    struct TileH {
        half8 k[NV];
        half8 v[NV];
        uint16_t m[NG][4];
    };
    struct TileF {
        floatx4 k[NV][2];
        floatx4 v[NV][2];
        uint16_t m[NG][4];
    };
    using Tile = std::conditional_t<KV32, TileF, TileH>;
    // The wavefront's f16 K tile in LDS: row r, 16-byte chunk c at chunk
    // c ^ f(r) of the row (f(r) = r mod 16 at hd 128, (r / 2) mod 8 at hd 64):
    // the 16 rows one MFMA operand read takes from one column of chunks fall
    // on 16 different bank groups.
    _Float16* const kt = reinterpret_cast<_Float16*>(lds_kt_raw) + wave * TP * D;
    float* const ktf = reinterpret_cast<float*>(lds_kt_raw) + wave * TP * D;
    auto kt_at = [](int r, int c) { return r * D + 8 * (c ^ ((D == 64 ? (r >> 1) : r) & (NCH - 1))); };
    auto vval = [&](const Tile& T, int i, int j) -> float {
        if constexpr (KV32) return T.v[i][j >> 2][j & 3];
        else return (float)T.v[i][j];
    };
    // cache row of logical position pos: pos itself, or in a ring of
    // ring_cap rows starting at ring_start, (ring_start + pos) mod ring_cap
    // (ring_cap = ring_start = 0 leaves pos unchanged)
    auto row_of = [&](int pos) {
        if constexpr (!RING) return pos;
        const int r = pos + a.ring_start;
        return r >= a.ring_cap ? r - a.ring_cap : r;
    };
    // K/V tiles are read once per step: nontemporal loads without a mask
    // tensor (f16, measured 12.65 -> 12.37 us per layer at n_kv 8192 on one
    // box, 12.66 -> 12.60 on another; F32 with 16-position tiles and F32
    // MFMA, 19.4 -> 18.7 us, likely also by leaving the split records in L2
    // for the combine); with one (the ragged batch) they measured ~1 %
    // slower, so masked f16 tiles keep ordinary loads
    // Addresses: a wave-uniform 64-bit row base (scalar registers) plus a
    // 32-bit lane offset, row * stride + column bytes by one 24-bit
    // multiply-add (the host keeps strides and ring sizes below 2^24 and a
    // ring's span below 2^31 bytes). Positions p0 + x of a tile clamp to its
    // last live position q: the tile's base row is that of position bp and
    // lane x reads row bp + min(x, lim), two VALU instructions per address.
    // In a ring (a template parameter, so a linear cache pays nothing for
    // it) a tile whose rows wrap takes the cache start as its base and
    // absolute rows as offsets.
    const uint32_t knb = (uint32_t)a.k_nb1, vnb = (uint32_t)a.v_nb1;
    auto load_tile = [&](Tile& T, int t) {
        const int p0 = lo + t * TP;
        const int q = min(p0 + TP, hi_main) - 1;
        const int bp = q >= p0 ? p0 : max(q, 0);
        const int lim = q >= p0 ? q - p0 : 0;
        const int rb = row_of(bp);
        bool wrap = false;
        if constexpr (RING) wrap = rb + lim >= a.ring_cap;
        auto row_off = [&](int x, uint32_t nb, int col) {
            const int rel = min(x, lim);
            int r = rel;
            if constexpr (RING) {
                const int ra = rb + rel >= a.ring_cap ? rb + rel - a.ring_cap : rb + rel;
                r = wrap ? ra : rel;
            }
            return __umul24((uint32_t)r, nb) + (uint32_t)col;
        };
        const char* ktile = wrap ? kb : kb + (int64_t)rb * a.k_nb1;
        const char* vt = wrap ? vb : vb + (int64_t)rb * a.v_nb1;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const char* kp = ktile + row_off(vrow + i * RPI, knb, vcol * ESZ);
            if constexpr (KV32) {
                T.k[i][0] = __builtin_nontemporal_load((const floatx4*)(kp));
                T.k[i][1] = __builtin_nontemporal_load((const floatx4*)(kp + 16));
            } else if constexpr (masked) {
                T.k[i] = *(const half8*)(kp);
            } else {
                T.k[i] = __builtin_nontemporal_load((const half8*)(kp));
            }
        }
#pragma unroll
        for (int grp = 0; grp < NG; ++grp) {
            if constexpr (masked) {
                const uint32_t pos = (uint32_t)(bp + min(16 * grp + (lane & 15), lim));
#pragma unroll
                for (int i = 0; i < 4; ++i) T.m[grp][i] = mplane[i][pos];
            }
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const char* vp = vt + row_off(vrow + i * RPI, vnb, vcol * ESZ);
            if constexpr (KV32) {
                T.v[i][0] = __builtin_nontemporal_load((const floatx4*)(vp));
                T.v[i][1] = __builtin_nontemporal_load((const floatx4*)(vp + 16));
            } else if constexpr (masked) {
                T.v[i] = *(const half8*)(vp);
            } else {
                T.v[i] = __builtin_nontemporal_load((const half8*)(vp));
            }
        }
    };

    // ---- prologue: Q and the first tile go out together -------------------
    // The group's G query heads (G * D elements, contiguous per head) are read
    // once per workgroup, 8 elements per thread, rounded to f16 (ggml's Q
    // conversion before an f16 K dot product; the MFMA product needs it for
    // F32 K too) and staged in LDS; each wavefront then reads its MFMA A
    // operand (head (lane & 15) % G, dims 32 ks + 8 (lane >> 4) .. + 7) from
    // there. (The Q element type is a template parameter: a load-or-convert
    // branch on it makes the compiler wait for all global loads inside the KV
    // loop.)
    constexpr int QCH = QF16 ? 1 : 2;                // 16-byte loads per 8 elements
    constexpr int QTHREADS = G * D / 8;              // threads holding 8 Q elements
    static_assert(QTHREADS <= DEC_THREADS, "Q staging");
    floatx4 qraw[QCH];
    const bool q_loader = tid < QTHREADS;
    {
        const int qh = g * G + (q_loader ? tid / (D / 8) : 0);
        const int qd = q_loader ? 8 * (tid % (D / 8)) : 0;
        const floatx4* p = (const floatx4*)((const char*)a.q + (int64_t)qh * a.q_nb2 + (int64_t)b * a.q_nb3 +
                                            (int64_t)qd * (QF16 ? 2 : 4));
#pragma unroll
        for (int u = 0; u < QCH; ++u) qraw[u] = p[u];
    }
    // The first tile's loads are unconditional (a wavefront without a tile
    // reads a clamped row it never uses): straight-line code lets the
    // compiler count the loads in flight exactly at the waits that follow.
    Tile TA, TB;
    int t = t_begin + wave;
    load_tile(TA, t < t_end ? t : t_begin);
    // the rotary cos / sin table, by wavefront 0 while the tile loads are in
    // flight; the q_loader lanes read it next, in program order. (The empty
    // asm takes the position as an operand after those loads are issued, so
    // the wait for it stays below them.)
    asm volatile("" : "+v"(rope_p) : : "memory");
    if (a.rope_pos && tid < D / 2) lds_rope[tid] = rope_cs_chain<D / 2>(rope_p, tid, a.rope_ts);
    half8* const lds_q = reinterpret_cast<half8*>(lds_q_raw);
    float* const lds_qf = reinterpret_cast<float*>(lds_q_raw);
    if (q_loader) {
        float x[8];
        if constexpr (!QF16) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = qraw[0][e];
                x[4 + e] = qraw[QCH - 1][e];
            }
            // rotary embedding of the query (position of batch b's token)
            if (a.rope_pos) rope8_tab(x, 8 * (tid % (D / 8)), lds_rope, a.rope_dims);
        }
        if constexpr (KV32) {
            // F32 K: Q stays F32 (ggml's F32 dot converts Q to F32, exactly)
            if constexpr (QF16) {
                const half8 qh = __builtin_bit_cast(half8, qraw[0]);
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = (float)qh[e];
            }
            *(floatx4*)(lds_qf + 8 * tid) = floatx4{x[0], x[1], x[2], x[3]};
            *(floatx4*)(lds_qf + 8 * tid + 4) = floatx4{x[4], x[5], x[6], x[7]};
        } else {
            half8 qh8;
            if constexpr (QF16) {
                qh8 = __builtin_bit_cast(half8, qraw[0]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) qh8[e] = (_Float16)x[e];
            }
            lds_q[tid] = qh8;
        }
    }
    __syncthreads();
    // MFMA A operands. f16 K: head (lane & 15) % G, dims 32 ks + 8 (lane / 16)
    // .. + 7 of step ks. F32 K (v_mfma_f32_16x16x4f32, one dim per lane and
    // step): lane l takes dim (D / 4) (l / 16) + s at step s, so its D / 4
    // values of Q (and of each K row) are contiguous.
    half8 qa[KS];
    float qf[KV32 ? D / 4 : 1];
    {
        const int m = (lane & 15) % G;
        if constexpr (KV32) {
#pragma unroll
            for (int cq = 0; cq < D / 16; ++cq) {
                const floatx4 v = *(const floatx4*)(lds_qf + m * D + (D / 4) * (lane >> 4) + 4 * cq);
#pragma unroll
                for (int e = 0; e < 4; ++e) qf[4 * cq + e] = v[e];
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qa[ks] = lds_q[(m * D + 32 * ks + 8 * (lane >> 4)) / 8];
        }
    }

    float m_run[4], l_run[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { m_run[i] = -INFINITY; l_run[i] = 0.f; }
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.f;

    auto process = [&](const Tile& T, int p0, int pend) {
        // K rows into the wavefront's LDS tile, MFMA B operands out (position
        // 16 grp + lane % 16, dims 32 ks + 8 (lane / 16) .. + 7). LDS
        // instructions of one wavefront execute in order, so its reads see
        // its writes; the previous tile's reads have returned (its MFMAs used
        // them) before these writes issue.
        floatx4 sc[NG];
        if constexpr (KV32) {
            // F32 rows, 16-byte chunk c of row r at chunk c ^ (r % 16): the 16
            // rows of one operand read (one chunk each) fall on 16 bank groups.
            // S^T in F32: v_mfma_f32_16x16x4f32, D / 4 steps, the products and
            // their sums in F32 as ggml's F32 dot (the matrix pipe has time to
            // spare in an HBM-bound kernel).
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int r = vrow + i * RPI, c0 = 2 * (lane % CH);
                *(floatx4*)(ktf + r * D + 4 * (c0 ^ (r & 15))) = T.k[i][0];
                *(floatx4*)(ktf + r * D + 4 * ((c0 + 1) ^ (r & 15))) = T.k[i][1];
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int grp = 0; grp < NG; ++grp) {
                const int r = 16 * grp + (lane & 15);
                sc[grp] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int cq = 0; cq < D / 16; ++cq) {
                    const floatx4 kv = *(const floatx4*)(ktf + r * D + 4 * (((D / 16) * (lane >> 4) + cq) ^ (r & 15)));
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        sc[grp] = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[4 * cq + e], kv[e], sc[grp], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) *(half8*)(kt + kt_at(vrow + i * RPI, lane % CH)) = T.k[i];
            __builtin_amdgcn_wave_barrier();
            half8 kop[NG][KS];
#pragma unroll
            for (int grp = 0; grp < NG; ++grp)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    kop[grp][ks] = *(const half8*)(kt + kt_at(16 * grp + (lane & 15), 4 * ks + (lane >> 4)));
#pragma unroll
            for (int grp = 0; grp < NG; ++grp) {
                sc[grp] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    sc[grp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[ks], kop[grp][ks], sc[grp], 0, 0, 0);
            }
        }
        // scores in log2 units; lane holds head (i % G) at position p0 + 16*grp + (lane & 15)
        float x[NG][4];
#pragma unroll
        for (int grp = 0; grp < NG; ++grp) {
            const bool valid = p0 + 16 * grp + (lane & 15) < pend;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float xv = sc[grp][i] * a.scale_log2;
                if constexpr (masked) {
                    const uint16_t mb = T.m[grp][i];
                    xv = (mb == kF16NegInf) ? -INFINITY : fmaf(f16_bits_to_f32(mb), kLog2e, xv);
                }
                x[grp][i] = valid ? xv : -INFINITY;
            }
        }
        float alpha[4], p[NG][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float mx = x[0][i];
#pragma unroll
            for (int grp = 1; grp < NG; ++grp) mx = fmaxf(mx, x[grp][i]);
            mx = row16_max(mx);
            const float mnew = fmaxf(m_run[i], mx);
            const float msafe = (mnew == -INFINITY) ? 0.f : mnew;
            alpha[i] = exp2_fast(m_run[i] - msafe);
            float ps = 0.f;
#pragma unroll
            for (int grp = 0; grp < NG; ++grp) {
                p[grp][i] = exp2_fast(x[grp][i] - msafe);
                ps += p[grp][i];
            }
            l_run[i] = fmaf(l_run[i], alpha[i], ps);
            m_run[i] = mnew;
        }
        if ((lane >> 4) == 0) {
#pragma unroll
            for (int grp = 0; grp < NG; ++grp)
                lds_p[wave][16 * grp + lane] = floatx4{p[grp][0], p[grp][1], p[grp][2], p[grp][3]};
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[h][j] *= alpha[h];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const floatx4 pv = lds_p[wave][vrow + i * RPI];
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(pv[h], vval(T, i, j), acc[h][j]);
        }
        __builtin_amdgcn_wave_barrier();
    };

    // ---- main loop: two register sets, the next tile loads during compute ----
    // (The next tile's loads sit under a branch, so at the join the compiler
    // counts loads in flight as on the path without them: in a walk of
    // several tiles each tile's V waits also wait for most of the next tile's
    // loads. Putting every process() on a straight path (the loop peeled
    // into three or four copies) removes those waits but raised the kernel
    // to 256 VGPRs + 48-107 AGPRs, one wavefront per SIMD, or with two forced
    // per SIMD to 60-420 bytes of scratch per lane: n_kv 8192 11.2 -> 13.1 us
    // per layer, 32 ragged streams 135 -> 146 us.)
    while (t < t_end) {
        int tn = t + DEC_WAVES;
        if (tn < t_end) load_tile(TB, tn);
        process(TA, lo + t * TP, min(lo + t * TP + TP, hi_main));
        t = tn;
        if (t >= t_end) break;
        tn = t + DEC_WAVES;
        if (tn < t_end) load_tile(TA, tn);
        process(TB, lo + t * TP, min(lo + t * TP + TP, hi_main));
        t = tn;
    }

    // ---- fused append: the new row, from the F32 sources --------------------
    // Every lane reads the new row in its own K and V operand layout (all
    // positions of the one-row tile clamp to it; only position n_kv - 1 is
    // valid in process()), rounded to f16 exactly as the cache will hold it.
    // The lanes holding each element once write the rounded row to the cache.
    // (f16 caches only; the host rejects an append to an F32 cache.)
    if constexpr (!KV32) {
        if (a.append && split == a.n_split - 1 && wave == 0) {
            const int pn = a.nkv - 1;
            const float* kn = (const float*)((const char*)a.k_new + (int64_t)bkv * a.kn_nb3) + g * D;
            const float* vn = (const float*)((const char*)a.v_new + (int64_t)bkv * a.vn_nb3) + g * D;
            // every load of the row first (one round trip), then rotation (K,
            // with rope_pos; the table holds the row's angles) and rounding
            floatx4 kr[2], vr[2];
            kr[0] = *(const floatx4*)(kn + vcol);
            kr[1] = *(const floatx4*)(kn + vcol + 4);
            vr[0] = *(const floatx4*)(vn + vcol);
            vr[1] = *(const floatx4*)(vn + vcol + 4);
            auto cvt8 = [&](const floatx4 (&r)[2], int d0, bool rot) {
                float x[8] = {r[0][0], r[0][1], r[0][2], r[0][3], r[1][0], r[1][1], r[1][2], r[1][3]};
                if (rot) rope8_tab(x, d0, lds_rope, a.rope_dims);
                half8 y;
#pragma unroll
                for (int i = 0; i < 8; ++i) y[i] = (_Float16)x[i];
                return y;
            };
            const bool rot = a.rope_pos != nullptr;
            const half8 kx = cvt8(kr, vcol, rot);
            const half8 vx = cvt8(vr, vcol, false);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                TA.k[i] = kx;
                TA.v[i] = vx;
            }
            if constexpr (masked) {
#pragma unroll
                for (int grp = 0; grp < NG; ++grp)
#pragma unroll
                    for (int i = 0; i < 4; ++i) TA.m[grp][i] = mplane[i][pn];
            }
            if (new_live) process(TA, pn, pn + 1);
            if (lane < CH) {
                *(half8*)((_Float16*)(kb + (int64_t)row_of(pn) * a.k_nb1) + vcol) = kx;
                *(half8*)((_Float16*)(vb + (int64_t)row_of(pn) * a.v_nb1) + vcol) = vx;
            }
        }
    }

    // ---- merge lanes, then wavefronts ------------------------------------
    // Each of the 8 G sums acc[h][j] (value v = 8 h + j) is reduced over the
    // lanes sharing lane % CH. For CH = 16 by two cross-lane swap rounds on
    // the VALU (no LDS round trips), four values per register at the end:
    //   v_permlane32_swap(a, b) -> {[a_lo, b_lo], [a_hi, b_hi]} (32-lane
    //   halves), summed: lanes 0-31 hold a partial of a, 32-63 one of b;
    //   v_permlane16_swap(a, b) -> {[a0, b0, a2, b2], [a1, b1, a3, b3]}
    //   (16-lane rows), summed: rows hold [a0+a1, b0+b1, a2+a3, b2+b3].
    // Register j then holds value 4 j + perm(r) in row r, perm = (0, 2, 1, 3),
    // and lane (r, c) stores it to slot 4 j + r, column c, of the wavefront's
    // [8 G][16] LDS block (value v sits in slot (v & ~3) | perm(v & 3)).
    float* const lds_sum = &lds_acc[0][0][0];
    auto perm2 = [](int x) { return ((x & 1) << 1) | ((x >> 1) & 1); };
    if constexpr (CH == 16) {
        constexpr int NVAL = 8 * G;
        float s1[NVAL / 2];
#pragma unroll
        for (int k = 0; k < NVAL / 2; ++k) {
            const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, acc[(2 * k) / 8][(2 * k) % 8]),
                                                            __builtin_bit_cast(int, acc[(2 * k + 1) / 8][(2 * k + 1) % 8]),
                                                            false, false);
            s1[k] = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
        }
#pragma unroll
        for (int j = 0; j < NVAL / 4; ++j) {
            const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, s1[2 * j]),
                                                            __builtin_bit_cast(int, s1[2 * j + 1]), false, false);
            lds_sum[(wave * NVAL + 4 * j + (lane >> 4)) * 16 + (lane & 15)] =
                __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
        }
    } else {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float s = acc[h][j];
#pragma unroll
                for (int m = CH; m < 64; m <<= 1) s += shfl_xor(s, m);
                acc[h][j] = s;
            }
        if (lane < CH) {
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) lds_acc[wave][h][lane * 8 + j] = acc[h][j];
        }
    }
    // wavefront w's sum for head h, dim d
    auto acc_at = [&](int w, int h, int d) {
        if constexpr (CH == 16) {
            const int v = 8 * h + (d & 7);
            return lds_sum[(w * 8 * G + ((v & ~3) | perm2(v & 3))) * 16 + (d >> 3)];
        } else {
            return lds_acc[w][h][d];
        }
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) l_run[i] = row16_sum(l_run[i]);

    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) { lds_m[wave][h] = m_run[h]; lds_l[wave][h] = l_run[h]; }
    }
    __syncthreads();

    float* rec = nullptr;
    if (a.n_split > 1)
        rec = a.ws + ((int64_t)(b * a.hkv + g) * a.n_split + split) * dec_record_floats(D, G);
    for (int o = tid; o < G * D; o += DEC_THREADS) {
        const int h = o / D, d = o % D;
        float M = lds_m[0][h];
#pragma unroll
        for (int w = 1; w < DEC_WAVES; ++w) M = fmaxf(M, lds_m[w][h]);
        const float Ms = (M == -INFINITY) ? 0.f : M;
        float s = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < DEC_WAVES; ++w) {
            const float wt = exp2_fast(lds_m[w][h] - Ms);
            s = fmaf(wt, acc_at(w, h, d), s);
            L = fmaf(wt, lds_l[w][h], L);
        }
        if (rec == nullptr) {
            a.dst[((int64_t)b * a.hq + g * G + h) * D + d] = (L == 0.f) ? 0.f : s / L;
        } else {
            rec[o] = s;
            if (d == 0) { rec[G * D + h] = M; rec[G * D + G + h] = L; }
        }
    }
}

template <int D, int G, bool KV32, bool T16>
static hipError_t launch_dgk(const AttnArgs& a, hipStream_t st) {
    const dim3 grid(a.n_split * a.hkv, a.b), block(DEC_THREADS);
    const DecodeDivs dv = {DivMod::make(a.hkv), DivMod::make(a.n_split), DivMod::make(a.b / a.bk),
                           DivMod::make(a.hm > 0 ? a.hm : 1), DivMod::make(a.bm > 0 ? a.bm : 1)};
    if (a.mask) {
        if (a.q_f16) hipLaunchKernelGGL((fa_decode<D, G, true, true, KV32, false, T16>), grid, block, 0, st, a, dv);
        else hipLaunchKernelGGL((fa_decode<D, G, false, true, KV32, false, T16>), grid, block, 0, st, a, dv);
    } else if (a.ring_cap > 0) {
        // a ring: f16 cache, no mask tensor (the host rejects anything else)
        if constexpr (!KV32) {
            if (a.q_f16) hipLaunchKernelGGL((fa_decode<D, G, true, false, false, true, T16>), grid, block, 0, st, a, dv);
            else hipLaunchKernelGGL((fa_decode<D, G, false, false, false, true, T16>), grid, block, 0, st, a, dv);
        }
    } else {
        if (a.q_f16) hipLaunchKernelGGL((fa_decode<D, G, true, false, KV32, false, T16>), grid, block, 0, st, a, dv);
        else hipLaunchKernelGGL((fa_decode<D, G, false, false, KV32, false, T16>), grid, block, 0, st, a, dv);
    }
    // the combine loads ceil(n_split / 8) partial slices per lane
    const dim3 cgrid(a.hkv * G * (D / 32), a.b);
    if (a.n_split > 32) hipLaunchKernelGGL((fa_decode_combine<D, G, 8>), cgrid, dim3(64), 0, st, a);
    else if (a.n_split > 16) hipLaunchKernelGGL((fa_decode_combine<D, G, 4>), cgrid, dim3(64), 0, st, a);
    else if (a.n_split > 8) hipLaunchKernelGGL((fa_decode_combine<D, G, 2>), cgrid, dim3(64), 0, st, a);
    else if (a.n_split > 1) hipLaunchKernelGGL((fa_decode_combine<D, G, 1>), cgrid, dim3(64), 0, st, a);
    return hipGetLastError();
}
template <int D, int G>
static hipError_t launch_dg(const AttnArgs& a, hipStream_t st) {
    if (a.kv_f32) return launch_dgk<D, G, true, false>(a, st);
    return a.dec_t16 ? launch_dgk<D, G, false, true>(a, st) : launch_dgk<D, G, false, false>(a, st);
}

hipError_t launch_decode(const AttnArgs& a, int head_dim, int group, hipStream_t st) {
    if (a.n_split < 1 || a.n_split > kDecodeMaxSplit) return hipErrorInvalidValue;
    if (a.n_split > 1 && a.ws == nullptr) return hipErrorInvalidValue;
    if (a.b > 65535 || (int64_t)a.n_split * a.hkv > 0x7fffffff) return hipErrorInvalidValue;
    if (a.kv_f32 && a.append) return hipErrorInvalidValue;
    if (a.ring_cap > 0 && (a.kv_f32 || a.mask)) return hipErrorInvalidValue;
    // the kernel's 32-bit lane offsets: row strides below 2^24 bytes; a ring
    // of fewer than 2^24 rows spanning less than 2^31 bytes
    if (a.k_nb1 < 0 || a.k_nb1 >= (1 << 24) || a.v_nb1 < 0 || a.v_nb1 >= (1 << 24)) return hipErrorInvalidValue;
    if (a.ring_cap > 0 && (a.ring_cap >= (1 << 24) ||
                           (int64_t)a.ring_cap * (a.k_nb1 > a.v_nb1 ? a.k_nb1 : a.v_nb1) >= ((int64_t)1 << 31)))
        return hipErrorInvalidValue;
    if (head_dim == 128) {
        if (group == 4) return launch_dg<128, 4>(a, st);
        if (group == 2) return launch_dg<128, 2>(a, st);
        if (group == 1) return launch_dg<128, 1>(a, st);
    } else if (head_dim == 64) {
        if (group == 4) return launch_dg<64, 4>(a, st);
        if (group == 2) return launch_dg<64, 2>(a, st);
        if (group == 1) return launch_dg<64, 1>(a, st);
    }
    return hipErrorInvalidValue;
}

__global__ void zero_kernel(float* dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = 0.f;
}

hipError_t launch_zero(float* dst, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, n);
    return hipGetLastError();
}

// F32 -> f16 (round to nearest even) copies of K and V for the prefill
// kernels, whose tiles reach LDS by direct global-to-LDS copies: one launch,
// blockIdx.y picks K or V (the staging body, stage_groups, is in fa_common.h).
template <bool NT>
__global__ __launch_bounds__(256) void to_f16_kv_kernel(StageArgs sa) {
    stage_groups<NT>(sa, blockIdx.x, (int)blockIdx.y, threadIdx.x);
}

hipError_t launch_to_f16_kv(const StageReq& r, hipStream_t st) {
    StageArgs sa;
    uint32_t blocks = 0;
    bool nt = false;
    if (!make_stage_args(r, sa, blocks, nt)) return hipErrorInvalidValue;
    if (sa.total8 == 0) return hipSuccess;
    const dim3 grid(blocks, 2);
    if (nt) hipLaunchKernelGGL(to_f16_kv_kernel<true>, grid, dim3(256), 0, st, sa);
    else hipLaunchKernelGGL(to_f16_kv_kernel<false>, grid, dim3(256), 0, st, sa);
    return hipGetLastError();
}

}  // namespace vxfa
