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
  * the s_waitcnt vmcnt(N) before a block's first read leaves only copies of
    later blocks in flight (vector-memory loads complete in issue order),
  * no copy is issued into a slot whose block still has reads to come.

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
# fa_prefill_pp.hip (Shape<NQT, KVG, NS>): a shared ring per KV group, one
# barrier per block; wavefront (kg, wq) copies rows 8 (NQT i + wq) + l / 8

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


def emulate_pp(sh: Shape, NQT=2, KVG=4, NS=4):
    BM = 64 * NQT
    NLD = 4 // NQT
    nqg = (sh.nq + BM - 1) // BM
    nblk = (sh.nkv + 31) // 32
    ni = (nblk + KVG - 1) // KVG
    AHEAD = NS - 1
    for kg in range(KVG):
        bs = min(kg * ni, nblk)
        ng = min(ni, nblk - bs)
        part = ng > 0 and (bs + ng) * 32 > sh.nkv
        nf = ng - (1 if part else 0)
        mems = []
        for wq in range(NQT):
            mem = Mem()
            for _ in range(BM * 16 // (64 * NQT * KVG)):
                mem.issue("Q")
            npre = min(ng, AHEAD)
            for blk in range(npre):
                pp_copy(sh, NQT, KVG, NS, kg, wq, bs, blk, mem)
            mem.wait(min(npre, 8) * 2 * NLD)
            _check(mem.complete("Q"), "Q staged before its loads completed")
            mem.wait(max(npre - 2, 0) * 2 * NLD)
            mems.append((mem, npre))
        # barrier: blocks 0 and 1 visible to every wavefront of the group
        for b0 in range(min(2, ng)):
            _check(all(m.complete(b0) for m, _ in mems), f"block {b0} not landed at the prologue barrier")
        for t in range(0, max(nf - 1, 0)):
            for wq, (mem, _) in enumerate(mems):
                if t + AHEAD < ng:
                    pp_copy(sh, NQT, KVG, NS, kg, wq, bs, t + AHEAD, mem)
                mem.wait(max(min(t + AHEAD, ng - 1) - (t + 2), 0) * 2 * NLD)
            # barrier; block t + 1 is read at the top of the next iteration and
            # must be complete in every wavefront's copies (t + 2 for the one after)
            for b1 in (t + 1, t + 2):
                if b1 < ng:
                    _check(all(m.complete(b1) for m, _ in mems), f"block {b1} not landed at barrier {t}")
            # the slot refilled at iteration t held block t - 1, last read in iteration t - 1
            if t + AHEAD < ng:
                _check((t + AHEAD) % NS == (t - 1) % NS or t == 0, "refill of a live slot")
        for mem, _ in mems:
            mem.wait(0)
    return {"nblk": nblk}
