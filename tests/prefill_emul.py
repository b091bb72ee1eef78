"""CPU emulation of the masked hd 128 prefill kernel's memory schedule
(voxtral.cpp_amd/csrc/fa_prefill.hip, fa_prefill_kernel<128, 2, 2, MM = 1>:
2 query wavefronts x 2 KV groups, two LDS stages of 128 positions), as it
ships and in the reordered form that issues step 0's K/V copies before the
mask scan (mask_scan_tiles).

Per workgroup it replays, wavefront by wavefront, every vector-memory
instruction in issue order -- the mask scan's loads, the Q loads its
after_loads hook issues, the LDS copies of each step (global_load_lds_dwordx4,
restated lane by lane: global row, 16-byte chunk, LDS target), the mask-word
loads of mixed tiles -- and every wait (the compiler's counted waits for the
loads it sees, wait_all_mem's vmcnt(0)), barrier and LDS access (the scan's
tile flags and reductions, the K and V operand reads of each step, the
KV-group merge that reuses the stage arrays, the end of each wavefront). With
vector-memory loads completing in issue order it checks that

  * every copy reads 16 bytes of an existing K or V row (rows past n_kv
    clamped) and lands inside its stage of sK / sV;
  * no LDS access (flag and reduction writes, operand reads, merge writes)
    touches bytes that a copy still in flight, from any wavefront of the
    workgroup, will write;
  * every step's copies have landed in every wavefront before its operands
    are read;
  * no wavefront ends with a copy in flight (the workgroup's LDS would be
    handed to the next workgroup while the copy still writes into it).

The LDS arrays are distinct objects (the compiler gives __shared__ arrays
disjoint ranges), so the model keeps one address space per array.
"""
from __future__ import annotations

import numpy as np

from dma_emul import LANES, Violation, _check

D, NQW, KVG = 128, 2, 2
NW = NQW * KVG
NT = 64 * NW
BM = 32 * NQW
BS = 64 * KVG
CH = D // 8
RPL = 64 // CH
NLOAD = BS * CH // NT
TILE = BS * D * 2
KS = D // 16
UB = 4
PF_MAXT = 512


def swz_k128(r):
    return ((r >> 1) ^ (r << 2)) & 15


def swz_v128(r):
    return (r & 2) << 1


class Wave:
    """One wavefront's vector-memory instructions in issue order."""

    def __init__(self, w):
        self.w = w
        self.ops = []            # (kind, tag, array, lo, hi) ; kind 'dma' or 'load'
        self.done = 0
        self.ended = False

    def issue(self, kind, tag, array=None, lo=0, hi=0):
        self.ops.append((kind, tag, array, lo, hi))

    def wait(self, n):
        """s_waitcnt vmcnt(n): all but the n youngest have completed."""
        self.done = max(self.done, len(self.ops) - n)

    def wait_for(self, tag):
        """The compiler's counted wait before using the loads tagged `tag`:
        it counts the younger loads it knows of (not the inline-asm copies),
        so it waits for vmcnt(known younger), which with copies issued after
        the loads completes more than it needs, never less."""
        idx = [i for i, op in enumerate(self.ops) if op[1] == tag]
        if not idx:
            return
        last = idx[-1]
        known_younger = sum(1 for op in self.ops[last + 1:] if op[0] == "load")
        self.wait(known_younger)
        _check(all(i < self.done for i in idx), f"wave {self.w}: {tag} used before it landed")

    def inflight_dma(self):
        return [op for op in self.ops[self.done:] if op[0] == "dma"]

    def landed(self, tag):
        return all(i < self.done for i, op in enumerate(self.ops) if op[1] == tag)


class WG:
    def __init__(self, nq, nkv, k_nb1, v_nb1, plant=None):
        self.nq, self.nkv, self.k_nb1, self.v_nb1 = nq, nkv, k_nb1, v_nb1
        self.waves = [Wave(w) for w in range(NW)]
        self.plant = plant

    # -- LDS accesses --------------------------------------------------------
    def lds(self, array, lo, hi, what):
        for wv in self.waves:
            for _, tag, arr, a, b in wv.inflight_dma():
                if arr == array and a < hi and lo < b:
                    raise Violation(f"{what} touches {array}[{lo}:{hi}] while copy {tag} of wave {wv.w} is in flight")

    def barrier(self):
        pass   # the model checks LDS accesses against copies in flight at the access

    # -- copies (issue_step) -------------------------------------------------
    def issue_step(self, wv, s, stg):
        w = wv.w
        kv0 = s * BS
        _check(0 <= kv0 < self.nkv, f"step {s} outside the KV range")
        full = kv0 + BS <= self.nkv
        for i in range(NLOAD):
            r0 = RPL * (w + NW * i)
            r = r0 + LANES // CH
            rows = kv0 + r if full else np.minimum(kv0 + r, self.nkv - 1)
            _check((rows >= 0) & (rows < self.nkv), "copy of a row outside K/V")
            for name, nb1, swz, arr in (("K", self.k_nb1, swz_k128, "sK"), ("V", self.v_nb1, swz_v128, "sV")):
                col = ((LANES % CH) ^ swz(r)) * 16
                _check((col >= 0) & (col + 16 <= 2 * D), "chunk outside the row")
                off = rows * nb1 + col
                _check(off + 16 <= self.nkv * nb1, "copy past the K/V view")
                dst = stg * TILE + r0 * D * 2 + 16 * LANES
                _check((dst >= stg * TILE) & (dst + 16 <= (stg + 1) * TILE), "copy outside its stage")
                wv.issue("dma", f"{name}{s}@{stg}", arr, int(dst.min()), int(dst.max()) + 16)


def _live_tiles(mask_fn, q0, nq, nkv):
    """tile classes of the workgroup's rows: per 32-row group and 64-position
    tile, 1 all zero, 2 all -inf, 3 mixed (the scan's flags), and the live
    range of steps."""
    rows = range(q0, min(q0 + BM, nq))
    ntile = (nkv + 63) // 64
    live = np.zeros(nkv, bool)
    flags = {}
    for g in range(NQW):
        grow = [r for r in rows if q0 + 32 * g <= r < q0 + 32 * g + 32]
        for t in range(ntile):
            cols = range(64 * t, min(64 * t + 64, nkv))
            vals = [mask_fn(r, cc) for r in grow for cc in cols]
            anylive = any(vals)
            if anylive:
                live[list(cols)] |= True
            flags[(g, t)] = 0 if not grow else (1 if all(vals) and len(cols) == 64 else (2 if not anylive else 3))
    idx = np.flatnonzero(live)
    if idx.size == 0:
        return flags, 0, 0
    return flags, idx[0] // BS, idx[-1] // BS + 1


def emulate_prefill_masked(nq, nkv, hkv=8, mask_fn=None, order="shipped", plant=None, q_f32=True):
    """Every workgroup of one (head, batch) of the masked hd 128 prefill.
    mask_fn(i, j) -> True where row i attends kv j (default: causal with
    n_kv - n_q cached rows). order: "shipped" (copies after the scan) or
    "copies_first" (step 0's copies issued before the scan; after it the
    first step is copied again only when it is not step 0).
    plant (tests only): "issue_after_wait" issues the first step's copies
    after the wait that should cover them, "same_stage" copies the next step into the stage being read,
    "prefetch_at_end" issues one more copy (a prefetch of the next head's
    first step) after the last wait, "past_nkv" copies one step past the
    live range."""
    if mask_fn is None:
        off = nkv - nq
        mask_fn = lambda i, j: j <= i + off
    k_nb1 = v_nb1 = hkv * D * 2
    nqt = (nq + BM - 1) // BM
    ntile = (nkv + 63) // 64
    for qt in range(nqt):
        q0 = qt * BM
        wg = WG(nq, nkv, k_nb1, v_nb1, plant)
        flags, step_lo, step_hi = _live_tiles(mask_fn, q0, nq, nkv)
        first = step_lo if step_lo < step_hi else -1
        # (0) reordered form: step 0's copies before the scan
        if order == "copies_first":
            for wv in wg.waves:
                wg.issue_step(wv, 0, 0)
        # (1) mask_scan_tiles: batch loads, the after_loads hook (Q), flags, reductions
        units = NQW * min(ntile, PF_MAXT)
        for wv in wg.waves:
            ub = wv.w * UB
            first_batch = True
            while ub < units or first_batch:
                if ub < units:
                    for _ in range(UB * 5):
                        wv.issue("load", f"mask{ub}")
                if first_batch:
                    for _ in range(2 * KS if q_f32 else KS):
                        wv.issue("load", "Q")
                    wv.issue("load", "Q")   # rotary position word (F32 Q)
                    first_batch = False
                if ub < units:
                    wv.wait_for(f"mask{ub}")
                    for i in range(UB):
                        u = ub + i
                        if u < units:
                            g, t = divmod(u, min(ntile, PF_MAXT))
                            wg.lds("s_tflag", g * PF_MAXT + t, g * PF_MAXT + t + 1, f"flag write of wave {wv.w}")
                ub += NW * UB
            wg.lds("s_red", 8 * wv.w, 8 * wv.w + 8, f"reduction write of wave {wv.w}")
        for wv in wg.waves:
            wg.lds("s_red", 0, 8 * NW, f"reduction read of wave {wv.w}")
        # (2) the first step, mixed-tile mask words, Q, wait, barrier
        copy_first = first >= 0 and not (order == "copies_first" and first == 0)
        if copy_first and plant != "issue_after_wait":
            for wv in wg.waves:
                wg.issue_step(wv, first, 0)
        for wv in wg.waves:
            kg, qw = divmod(wv.w, NQW)
            if first >= 0 and first * BS + 64 * kg < nkv and flags.get((qw, (first * BS + 64 * kg) // 64)) == 3:
                wv.issue("load", f"mw{first}")
            wv.wait_for("Q")
            wv.wait(0)
        if copy_first and plant == "issue_after_wait":
            for wv in wg.waves:
                wg.issue_step(wv, first, 0)
        # (3) the steps
        seq = list(range(first, step_hi)) if first >= 0 else []
        if plant == "past_nkv" and seq:
            seq.append((nkv + BS - 1) // BS)
        for n, s in enumerate(seq):
            stg = n % 2
            nxt = seq[n + 1] if n + 1 < len(seq) else -1
            for wv in wg.waves:
                kg, qw = divmod(wv.w, NQW)
                if nxt >= 0:
                    wg.issue_step(wv, nxt, stg if plant == "same_stage" else stg ^ 1)
                    kv0n = nxt * BS + 64 * kg
                    if kv0n < nkv and flags.get((qw, kv0n // 64)) == 3:
                        wv.issue("load", f"mw{nxt}")
            for wv in wg.waves:
                kg, qw = divmod(wv.w, NQW)
                kv0 = s * BS + 64 * kg
                if kv0 >= nkv:
                    continue
                f = flags.get((qw, kv0 // 64), 3)
                wg.lds("s_tflag", qw * PF_MAXT + kv0 // 64, qw * PF_MAXT + kv0 // 64 + 1, "tile class read")
                if f in (1, 3):
                    if f == 3:
                        wv.wait_for(f"mw{s}")
                    for other in wg.waves:
                        _check(other.landed(f"K{s}@{stg}") and other.landed(f"V{s}@{stg}"),
                               f"step {s} read before wave {other.w}'s copies landed")
                    lo = stg * TILE + 64 * kg * D * 2
                    wg.lds("sK", lo, lo + 64 * D * 2, f"K operand reads of step {s}")
                    wg.lds("sV", lo, lo + 64 * D * 2, f"V operand reads of step {s}")
            last = n + 1 == len(seq)
            for wv in wg.waves:
                if not (plant == "no_final_wait" and last):
                    wv.wait(0)
        if plant == "prefetch_at_end" and seq:
            for wv in wg.waves:
                wg.issue_step(wv, seq[0], 0)
        # (4) merge: groups 1.. publish O into sV then sK, and (m, l) into s_ml
        for wv in wg.waves:
            kg, _ = divmod(wv.w, NQW)
            if kg > 0:
                wg.lds("sV", 0, 2 * TILE, f"merge write of wave {wv.w}")
                wg.lds("sK", 0, 2 * TILE, f"merge write of wave {wv.w}")
        for wv in wg.waves:
            kg, _ = divmod(wv.w, NQW)
            if kg > 0:
                _check(not wv.inflight_dma(), f"wave {wv.w} ends with copies in flight")
            else:
                wg.lds("sV", 0, 2 * TILE, f"merge read of wave {wv.w}")
        for wv in wg.waves:
            _check(not wv.inflight_dma(), f"wave {wv.w} ends with copies in flight")
    return True
