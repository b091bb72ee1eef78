"""CPU emulation of the global -> LDS copy schedule of the hd 64 encoder kernel.

Restates, lane by lane, the address arithmetic and the wait accounting of
voxtral.cpp_amd/csrc/fa_prefill_pp.hip (KVG groups x NQT query tiles, a
shared NS-slot ring per group, one barrier per block), so that a CPU test can
show, for a given shape and stride set, that

  * every global_load_lds_dwordx4 reads 16 bytes inside an existing K or V
    row (lane offset + scalar base, rows past n_kv clamped),
  * every copy lands inside its ring slot (M0 + 16 * lane) and inside the
    workgroup's LDS allocation,
  * every operand read from LDS (K 128-bit reads, V^T transposed 8-byte
    reads) stays inside the slot of the block it reads,
  * every block is landed, in both wavefronts' halves, at the barrier
    before the epoch that reads it (s_waitcnt vmcnt(N) leaves only younger
    copies in flight: vector-memory loads complete in issue order),
  * no copy is issued into a slot whose block still has reads to come (a
    copy in epoch e may overwrite a block last read in an earlier epoch),
  * every wavefront passes the same number of barriers.

Nothing here runs on a GPU; the formulas are the kernels' own, so a change to
a kernel's indexing has to be mirrored here for the test to stay meaningful.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

LANES = np.arange(64)


def swz_k64(r):
    return (r ^ (r >> 2)) & 7


def swz_v64(r):
    return (r & 2) << 1


@dataclass
class Shape:
    nq: int
    nkv: int
    hq: int
    hkv: int
    b: int = 1
    bk: int = 1
    k_nb1: int = 0      # bytes; default: [n][hkv][64] f16 rows
    v_nb1: int = 0
    k_nb2: int = 128
    v_nb2: int = 128

    def __post_init__(self):
        if not self.k_nb1:
            self.k_nb1 = self.hkv * 128
        if not self.v_nb1:
            self.v_nb1 = self.hkv * 128
        self.k_nb3 = self.k_nb1 * self.nkv
        self.v_nb3 = self.v_nb1 * self.nkv


class Violation(AssertionError):
    pass


def _check(cond, msg):
    if not np.all(cond):
        raise Violation(msg)


def _row_bytes_ok(off, nb1, nkv, base_row):
    """16-byte chunk at byte `off` from row `base_row`'s start lies inside a
    row < nkv and inside that row's 128 data bytes."""
    row = base_row + off // nb1
    within = off % nb1
    return (row < nkv) & (row >= 0) & (within + 16 <= 128) & (within % 16 == 0)


class Mem:
    """In-order completion model of one wavefront's vector-memory loads."""

    def __init__(self):
        self.log = []          # tags of issued load instructions
        self.done = 0          # the first `done` instructions have completed

    def issue(self, tag):
        self.log.append(tag)

    def wait(self, n):
        self.done = max(self.done, len(self.log) - n)

    def complete(self, tag):
        return all(i < self.done for i, t in enumerate(self.log) if t == tag)


# ---------------------------------------------------------------------------
# fa_prefill_pp.hip: KVG groups x NQT query tiles, an NS-slot ring per group;
# wavefront (kg, wq) copies rows 8 (NQT i + wq) + l / 8 of each block

def pp_copy(sh: Shape, NQT, KVG, NS, kg, wq, bs, blk, mem: Mem):
    BLK = 32 * 128
    GRP = 2 * BLK
    SLOT = KVG * GRP
    NLD = 4 // NQT
    kv0 = (bs + blk) * 32
    kd = kg * GRP + (blk % NS) * SLOT
    vd = kd + BLK
    full = kv0 + 32 <= sh.nkv
    rmax = sh.nkv - 1 - kv0
    _check(kv0 < sh.nkv, "copy of a block past n_kv")
    for i in range(NLD):
        r0 = 8 * (NQT * i + wq)
        r = r0 + (LANES >> 3)
        rc = r if full else np.minimum(r, rmax)
        for nb1, swz, dst, tag in ((sh.k_nb1, swz_k64, kd, "K"), (sh.v_nb1, swz_v64, vd, "V")):
            off = rc * nb1 + ((LANES & 7) ^ swz(r)) * 16
            _check(off < 2 ** 32, "32-bit lane offset overflow")
            _check(_row_bytes_ok(off, nb1, sh.nkv, kv0), f"{tag} copy reads outside the rows")
            lds = dst + r0 * 128 + 16 * LANES
            _check((lds >= dst) & (lds + 16 <= dst + BLK), "copy lands outside its block")
            _check(lds + 16 <= NS * SLOT, "copy lands outside the ring")
            mem.issue(blk)


def pp_block_range(sh: Shape, qg, BM=128, window=None, offset=0):
    """Blocks [blo, blo + nblk) the workgroup of query tile qg walks: all of
    them without a mask; under an implicit causal mask (window None: none,
    0: no lower bound) the blocks holding its rows' live positions
    i + offset - window < j <= i + offset (the kernel's formula)."""
    if window is None:
        return 0, (sh.nkv + 31) // 32
    qw0 = qg * BM
    q1 = min(qw0 + BM, sh.nq) - 1
    lo = qw0 + offset - window + 1 if window > 0 else 0
    hi = q1 + offset + 1
    lo, hi = max(lo, 0), min(hi, sh.nkv)
    if hi <= lo:
        lo = hi = 0
    blo = lo // 32
    return blo, (hi + 31) // 32 - blo


NEG_INF_F16 = 0xFC00


def mask_row_interval(row, mis):
    """The pre-pass of a mask tensor (mask_rows_kernel) for one F16 mask row
    (uint16 array of n entries) whose first entry sits mis bytes (even, < 16)
    past a 16-byte boundary: the row's 64 lanes read 16-byte chunks from the
    boundary, lane s of round c0 (c0 = 0, 192, ... below nchmax, the chunk
    count of the worst alignment) chunk min(c0 + 64 u + s, nch - 1) for
    u < 3, entry e of chunk slot c being column 8 c - mis / 2 + e; the
    entries of
    [elo, ehi) (those in [0, n)) count, through bit masks: live (in the row,
    not -inf) and nz (live and non-zero). From the first and last live
    columns lo and hi, their count and whether one is non-zero it returns
    (lo, hi) when the row is +-0 on [lo, hi] and -inf elsewhere (count
    hi - lo + 1, none non-zero), (n, -1) when every entry is -inf, (-2, -2)
    otherwise."""
    n = len(row)
    nch = (mis + 2 * n + 15) // 16
    nchmax = (14 + 2 * n + 15) // 16
    _check(nch <= nchmax, "the row has more chunks than the loop walks")
    lo, hi, cnt, nonzero = 1 << 31, -1, 0, False
    counted = []
    for c0 in range(0, nchmax, 64 * 3):
        for u in range(3):
            for s in range(64):
                c = c0 + 64 * u + s
                ld = min(c, nch - 1)             # the chunk the lane loads
                _check(0 <= ld < nch, "a load outside the row's chunks")
                col0 = 8 * c - mis // 2
                elo, ehi = max(-col0, 0), min(n - col0, 8)
                valid = ((1 << ehi) - 1) & ~((1 << elo) - 1) if ehi > elo else 0
                _check(c == ld or valid == 0, "a reloaded chunk counts")
                live = nz = 0
                for e in range(8):
                    if not (valid >> e) & 1:
                        continue
                    v = int(row[col0 + e])
                    l = v != NEG_INF_F16
                    live |= l << e
                    nz |= (l and (v & 0x7FFF) != 0) << e
                    counted.append(col0 + e)
                nonzero = nonzero or nz != 0
                if live:
                    first = col0 + (live & -live).bit_length() - 1
                    last = col0 + live.bit_length() - 1
                    lo, hi, cnt = min(lo, first), max(hi, last), cnt + bin(live).count("1")
    _check(sorted(counted) == list(range(n)), "the chunks miss or repeat a column")
    if hi < lo:
        return (n, -1)
    return (-2, -2) if nonzero or cnt != hi - lo + 1 else (lo, hi)


def pp_block_range_table(sh: Shape, qg, table, BM=128):
    """Blocks [blo, blo + nblk) the workgroup of query tile qg walks under a
    mask tensor (the kernel's MM = 1 logic): with any row of class (-2, -2)
    among its rows, every block; else the blocks between the smallest lo and
    the largest hi of its rows' intervals (none when all are empty). Rows
    past n_q count as empty. table: the pre-pass output of the rows of one
    (plane, batch)."""
    ivl = [tuple(table[r]) if r < sh.nq else (sh.nkv, -1) for r in range(qg * BM, qg * BM + BM)]
    if any(v[0] == -2 for v in ivl):
        return 0, (sh.nkv + 31) // 32
    live = [v for v in ivl if 0 <= v[0] <= v[1]]
    if not live:
        return 0, 0
    wlo, whi = min(v[0] for v in live), max(v[1] for v in live)
    blo = wlo // 32
    return blo, (whi + 32) // 32 - blo


def emulate_pp(sh: Shape, NQT=2, KVG=4, NS=4, plant=None, window=None, offset=0, table=None):
    """The kernel's copy schedule, epoch by epoch (epoch e runs between
    barrier e and barrier e + 1; the prologue's barrier is barrier 0 and
    iteration t of the main loop runs in epoch t), for every workgroup's
    block range (one range for all without a mask, see pp_block_range; a
    mask tensor's pre-pass table: pp_block_range_table).

    plant (tests only): "wait_late" waits for one block fewer at the end of
    each iteration, "copy_early" copies block t + NS + 1 in iteration t."""
    BM = 64 * NQT
    if table is not None:
        ranges = {pp_block_range_table(sh, qg, table, BM) for qg in range((sh.nq + BM - 1) // BM)}
    else:
        ranges = {pp_block_range(sh, qg, BM, window, offset) for qg in range((sh.nq + BM - 1) // BM)}
    for blo, nblk in sorted(ranges):
        _emulate_pp_range(sh, NQT, KVG, NS, plant, blo, nblk)
    return {"nblk": (sh.nkv + 31) // 32, "ranges": sorted(ranges)}


def _emulate_pp_range(sh: Shape, NQT, KVG, NS, plant, blo, nblk):
    BM = 64 * NQT
    NLD = 4 // NQT
    ni = (nblk + KVG - 1) // KVG
    ahead = NS + 1 if plant == "copy_early" else NS
    slack = 1 if plant == "wait_late" else 0
    _check(blo >= 0 and (blo + nblk) * 32 < sh.nkv + 32, "block range past n_kv")
    for kg in range(KVG):
        bs = blo + min(kg * ni, nblk)
        ng = min(ni, blo + nblk - bs)
        part = ng > 0 and (bs + ng) * 32 > sh.nkv
        nf = ng - (1 if part else 0)
        mems = [Mem() for _ in range(NQT)]
        copy_epoch = {}                      # block -> epoch its copies were issued in
        done_by = [dict() for _ in range(NQT)]   # block -> barrier by which this wavefront's copy had landed
        reads = []                           # (epoch, block)
        nbar = 0

        def copy(blk, epoch):
            for wq in range(NQT):
                pp_copy(sh, NQT, KVG, NS, kg, wq, bs, blk, mems[wq])
            _check(blk not in copy_epoch, f"block {blk} copied twice")
            copy_epoch[blk] = epoch

        def wait_all(k):                     # every wavefront: at most k blocks in flight
            for mem in mems:
                mem.wait(k * 2 * NLD)

        def barrier():
            nonlocal nbar
            for wq in range(NQT):
                for blk in copy_epoch:
                    if blk not in done_by[wq] and mems[wq].complete(blk):
                        done_by[wq][blk] = nbar
            nbar += 1

        # prologue: Q, then blocks 0 .. NS - 2
        npre = min(ng, NS - 1)
        for mem in mems:
            for _ in range(BM * 16 // (64 * NQT * KVG)):
                mem.issue("Q")
        for blk in range(npre):
            copy(blk, -1)
        for mem in mems:
            mem.wait(min(npre, 8) * 2 * NLD)
            _check(mem.complete("Q"), "Q staged before its loads completed")
        wait_all(max(npre - 2, 0))
        barrier()                            # barrier 0
        if nf > 0:
            reads += [(0, 0), (0, 0)]        # K_0, V_0
        for t in range(nf - 1):              # epoch t
            if t == 1 and NS < ng:
                copy(NS, t)
            reads.append((t, t + 1))         # K_{t+1}
            mid = NS - 1 if t == 0 else t + ahead
            if mid < ng:
                copy(mid, t)
            reads.append((t, t + 1))         # V_{t+1}
            last = min(t + ahead if t >= 1 else NS - 1, ng - 1)
            wait_all(max(last - (t + 2) + slack, 0))
            barrier()
        if nf > 0:
            wait_all(0)
            barrier()
        if part:
            reads += [(nbar - 1, nf)] * 2       # after the barrier that ends the last full block
            barrier()
        for _ in range(ng, ni):
            barrier()
        _check(nbar == 1 + ni, "barrier count differs from 1 + ni")
        for epoch, blk in reads:
            # both halves landed before the barrier that opened the epoch
            for wq in range(NQT):
                _check(done_by[wq].get(blk, 10 ** 9) <= epoch, f"block {blk} read in epoch {epoch} before it landed")
            # the slot still holds the block: the slot's next block is copied
            # in a later epoch
            nxt = blk + NS
            if nxt in copy_epoch:
                _check(copy_epoch[nxt] > epoch, f"block {blk} overwritten before its read in epoch {epoch}")
        _check(len(copy_epoch) == ng, "not every block of the group was copied")
