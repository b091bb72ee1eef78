"""CPU restatement of the addressing and work assignment of the short masked
prefill kernel (voxtral.cpp_amd/csrc/fa_prefill_pair.hip).

For a given shape, stride set and mask it shows, lane by lane, that

  * every Q load reads 16 bytes inside an existing query row,
  * every mask chunk read is a 16-byte-aligned granule holding at least one
    byte of its mask row (rows past n_q read row 0), and the words extracted
    from the three chunks (funnel shift by the row's misalignment, lane half
    1's halves swapped, -inf past n_kv and for rows past n_q) equal the mask
    entries at the positions the accumulator layout assigns to the lane,
  * every global -> LDS copy of a K or V tile reads 16 bytes inside an
    existing row (rows past n_kv clamped) and lands inside the LDS area, every
    byte of a used tile is written exactly once, and every K operand read and
    transposed V^T read of a computed block finds the global chunk it needs,
  * the assignment computes every live (query tile, KV tile) block exactly
    once and no dead one, and the merge stores every output element of every
    valid query row exactly once.

The formulas are the kernel's own, so a change to its indexing has to be
mirrored here for the test to stay meaningful. Nothing here runs on a GPU.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

D, KS, DB, TK, MAXK, NW = 128, 8, 4, 64, 8, 8
ROW, VT, QT = 256, 64 * 256, 32 * 256
LANES = np.arange(64)
NEG_INF = 0xFC00


class Violation(AssertionError):
    pass


def _check(cond, msg):
    if not np.all(cond):
        raise Violation(msg)


def pf_kv_of(hh, j):
    hh = np.asarray(hh)
    j = np.asarray(j)
    return np.where(hh != 0, 16 + (((j >> 2) + 2) & 3) * 4 + (j & 3), j)


def swz_v(r):
    return (np.asarray(r) & 3) << 2


def swz_k(r):
    r = np.asarray(r)
    return ((r >> 1) ^ (r << 2)) & 15


@dataclass
class Shape:
    nq: int
    nkv: int
    hq: int = 32
    hkv: int = 8
    b: int = 1
    bk: int = 1
    mode: str = "tensor"          # "tensor", "intervals" (tensor, classes from the pre-pass) or "implicit"
    offset: int = 0               # implicit mask: row i attends j <= i + offset
    window: int = 0               #   and j >= i + offset - window + 1 when window > 0
    m_nb1: int = 0                # mask row stride in bytes (default 2 n_kv: unpadded rows)
    m_mis: int = 0                # mask base misalignment in bytes (even)
    hm: int = 1
    bm: int = 1
    q_f16: bool = False
    kv_rows: int = 0              # cache rows allocated (>= n_kv)
    mask: np.ndarray = field(default=None, repr=False)   # uint16 [bm][hm][nq][nkv] (tensor mode)

    def __post_init__(self):
        if not self.m_nb1:
            self.m_nb1 = 2 * self.nkv
        if not self.kv_rows:
            self.kv_rows = self.nkv
        self.qe = 2 if self.q_f16 else 4
        # q: [B][Nq][Hq][D] rows; k, v: token-major cache [Bk][rows][Hkv][D] f16
        self.q_nb1, self.q_nb2 = self.hq * D * self.qe, D * self.qe
        self.q_nb3 = self.q_nb1 * self.nq
        self.k_nb1, self.k_nb2 = self.hkv * D * 2, D * 2
        self.k_nb3 = self.k_nb1 * self.kv_rows
        self.m_nb2 = self.m_nb1 * self.nq
        self.m_nb3 = self.m_nb2 * self.hm
        if self.mode != "implicit" and self.mask is None:
            i = np.arange(self.nq)[:, None]
            j = np.arange(self.nkv)[None, :]
            causal = np.where(j <= i + self.offset, 0, NEG_INF).astype(np.uint16)
            self.mask = np.broadcast_to(causal, (self.bm, self.hm, self.nq, self.nkv)).copy()

    # byte extents of the allocations (base 0 each; the mask at m_mis)
    def q_bytes(self):
        return self.q_nb3 * self.b

    def kv_bytes(self):
        return self.k_nb3 * self.bk

    def mask_buffer(self):
        """The mask tensor's bytes as the kernel sees them: entry (b, h, i, j)
        at m_mis + b m_nb3 + h m_nb2 + i m_nb1 + 2 j, the rest filled with a
        pattern that is never -inf or 0."""
        n = self.m_mis + self.m_nb3 * self.bm
        buf = np.full(n // 2 + 8, 0x3C01, dtype=np.uint16)   # 1.0009..., padded
        byts = buf.view(np.uint8)
        for bb in range(self.bm):
            for hh in range(self.hm):
                for i in range(self.nq):
                    o = self.m_mis + bb * self.m_nb3 + hh * self.m_nb2 + i * self.m_nb1
                    byts[o:o + 2 * self.nkv] = self.mask[bb, hh, i].view(np.uint8)
        return byts[:n]


def cls_formula(sh: Shape, T, j):
    r0, r1 = 32 * T, min(32 * T + 32, sh.nq) - 1
    c0, c1 = TK * j, min(TK * j + TK, sh.nkv) - 1
    if r1 < r0 or c1 < c0:
        return 0
    off, W = sh.offset, sh.window
    if c0 > r1 + off or (W > 0 and c1 < r0 + off - W + 1):
        return 0
    all_ = c1 <= r0 + off and (W == 0 or c0 >= r1 + off - W + 1)
    return 1 if (all_ and TK * j + TK <= sh.nkv) else 3


def mask_words_expected(sh: Shape, mplane_entry, T, j):
    """[64 lanes][2][8] words the lane should hold for block (T, j): mask
    entries at the accumulator positions, -inf past n_kv and for rows past
    n_q. mplane_entry(row, pos) -> uint16."""
    out = np.zeros((64, 2, 8), dtype=np.uint32)
    for lane in range(64):
        nl, hh = lane & 31, lane >> 5
        row = 32 * T + nl
        for kvb in range(2):
            for w in range(8):
                word = 0
                for e in range(2):
                    kv = TK * j + 32 * kvb + int(pf_kv_of(hh, 2 * w + e))
                    if row >= sh.nq or kv >= sh.nkv:
                        bits = NEG_INF
                    else:
                        bits = int(mplane_entry(row, kv))
                    word |= bits << (16 * e)
                out[lane, kvb, w] = word
    return out


def mask_words_interval(sh: Shape, table, T, j, plant=None):
    """The kernel's mw_interval (MM = 3, a tile whose rows are all intervals):
    lane (nl, hh) forms its words from row 32 T + nl's interval {lo, hi}
    (row min(., n_q - 1) for rows past n_q): 0 where lo <= kv <= hi and
    kv < n_kv, -inf elsewhere."""
    out = np.zeros((64, 2, 8), dtype=np.uint32)
    for lane in range(64):
        nl, hh = lane & 31, lane >> 5
        lo, hi = table[min(32 * T + nl, sh.nq - 1)]
        if plant == "interval_words_hi_open":
            hi += 1
        for kvb in range(2):
            for w in range(8):
                word = 0
                for e in range(2):
                    kv = TK * j + 32 * kvb + int(pf_kv_of(hh, 2 * w + e))
                    live = kv < sh.nkv and lo <= kv <= hi
                    word |= (0 if live else NEG_INF) << (16 * e)
                out[lane, kvb, w] = word
    return out


def mask_tile(sh: Shape, plane_off, T):
    """The kernel's mtile: tile T's first mask row rounded down to 16 bytes
    (the scalar base) and that row's offset from it."""
    t0 = plane_off + 32 * T * sh.m_nb1
    return t0 - (t0 & 15), t0 & 15


def mask_words_kernel(sh: Shape, buf, plane_off, T, j, plant=None):
    """The kernel's mw_issue + mw_finish, lane by lane, on the mask bytes:
    32-bit offsets from the tile's 16-byte-aligned base; checks every chunk
    address and returns the extracted words."""
    out = np.zeros((64, 2, 8), dtype=np.uint32)
    base16, d0 = mask_tile(sh, plane_off, T)
    for lane in range(64):
        nl, hh = lane & 31, lane >> 5
        row = 32 * T + nl
        rs = d0 + (nl if row < sh.nq else 0) * sh.m_nb1
        _check(0 <= rs < 2**31, "mask row offset beyond 32 bits")
        rowp = base16 + rs
        last = (rs + 2 * sh.nkv - 1) & ~15
        for kvb in range(2):
            segr = rs + 2 * (TK * j + 32 * kvb + 16 * hh)
            s = segr & 15
            pr = segr & ~15
            lim = last - pr
            chunks = []
            for i in range(3):
                off = 16 * i if plant == "no_chunk_clamp" else min(16 * i, lim)
                a = base16 + pr + off
                _check(a % 16 == 0, f"mask chunk not 16-byte aligned: {a}")
                # the granule [a, a + 16) must hold a byte of the row's data
                _check(a < rowp + 2 * sh.nkv and a + 16 > rowp,
                       f"mask chunk {a} outside row data [{rowp}, {rowp + 2 * sh.nkv}) (T {T}, j {j}, lane {lane})")
                _check(a >= 0 and a + 16 <= len(buf) + 16, "mask chunk outside the buffer")
                c = np.zeros(16, dtype=np.uint8)
                n = max(0, min(16, len(buf) - a))
                c[:n] = buf[a:a + n]
                chunks.append(c.view(np.uint32))
            d = np.concatenate(chunks)
            q4, s2 = s >> 2, s & 2
            e = [int(d[k + q4]) for k in range(9)]
            wv = []
            for k in range(8):
                v = ((e[k + 1] << 32) | e[k]) >> (8 * s2)
                wv.append(v & 0xFFFFFFFF)
            for w in range(8):
                out[lane, kvb, w] = wv[(w + 4) & 7] if hh else wv[w]
        if row >= sh.nq:
            out[lane] = 0xFC00FC00
        elif TK * j + TK > sh.nkv:
            for kvb in range(2):
                for w in range(8):
                    for e2 in range(2):
                        if TK * j + 32 * kvb + int(pf_kv_of(hh, 2 * w + e2)) >= sh.nkv:
                            word = int(out[lane, kvb, w])
                            word = (word & (0xFFFF0000 >> (16 * e2))) | (NEG_INF << (16 * e2))
                            out[lane, kvb, w] = word
    return out


def classify_kernel(sh: Shape, buf, plane_off, T, j, plant=None):
    """The kernel's cls_issue + cls_eval: each candidate row's 128-byte
    segment read as 16-byte-aligned chunks, nine lanes per row, seven rows per
    load, five loads; checks every chunk address, returns the class."""
    live = nonzero = False
    base16, d0 = mask_tile(sh, plane_off, T)
    for u in range(5):
        for lane in range(64):
            lr, lc = lane // 9, lane % 9
            rr = 7 * u + lr
            ok = lr < 7 and rr < 32 and 32 * T + rr < sh.nq
            rs = d0 + (rr * sh.m_nb1 if ok else 0)
            _check(0 <= rs < 2**31, "mask row offset beyond 32 bits")
            rowp = base16 + rs
            last = (rs + 2 * sh.nkv - 1) & ~15
            pr = (rs + 2 * TK * j) & ~15
            lim = last - pr
            a = base16 + pr + (16 * lc if plant == "no_chunk_clamp" else min(16 * lc, lim))
            _check(a % 16 == 0, "classification chunk not 16-byte aligned")
            _check(a < rowp + 2 * sh.nkv and a + 16 > rowp,
                   f"classification chunk {a} outside row data [{rowp}, {rowp + 2 * sh.nkv})")
            c = np.zeros(16, dtype=np.uint8)
            n = max(0, min(16, len(buf) - a))
            c[:n] = buf[a:a + n]
            w16 = c.view(np.uint16)
            e0 = (pr - rs + 16 * lc) // 2 if ok else 1 << 20
            lo, hi = max(TK * j - e0, 0), min(min(TK * j + TK, sh.nkv) - e0, 8)
            if hi <= lo:
                continue
            for k in range(lo, hi):
                v = int(w16[k])
                live |= v != NEG_INF
                nonzero |= (v & 0x7FFF) != 0
    if not live:
        return 0
    return 3 if (nonzero or TK * j + TK > sh.nkv) else 1


_TABLES = {}   # the pre-pass table of each (shape, plane), made once


def interval_table(sh: Shape, bb, h):
    """The mask pre-pass's table for the rows of plane (h % hm, bb % bm)
    (dma_emul.mask_row_interval of each row at its 16-byte alignment)."""
    from dma_emul import mask_row_interval
    out = []
    for i in range(sh.nq):
        off = sh.m_mis + (bb % sh.bm) * sh.m_nb3 + (h % sh.hm) * sh.m_nb2 + i * sh.m_nb1
        out.append(mask_row_interval(sh.mask[bb % sh.bm, h % sh.hm, i], off % 16))
    return out


def classify_intervals(sh: Shape, table, tA, tB, hasA, nk, plant=None):
    """The kernel's MM = 3 block classes, from the rows' intervals: per block
    j < nk of tile T, live when a real row's interval meets [64 j, 64 j + 64)
    (within n_kv) or a real row is not an interval (-2), all-zero when every
    real row's interval holds the block and the block lies within n_kv,
    mixed otherwise; rows past n_q take no part. Tile A only when it exists."""
    cls = {}
    for s_, T in ((0, tA), (1, tB)):
        if s_ == 0 and not hasA:
            continue
        for j in range(nk):
            c0, c1 = TK * j, min(TK * j + TK, sh.nkv) - 1
            live, cov = False, True
            for r in range(32):
                row = 32 * T + r
                if row >= sh.nq:
                    continue
                lo, hi = table[row]
                meets = lo <= c1 and hi >= c0
                holds = lo <= c0 and (hi >= c1 or plant == "holds_ignores_hi") and lo >= 0
                live = live or (lo == -2 and plant != "non_interval_dead") or meets
                cov = cov and lo != -2 and holds
            full = cov and TK * j + TK <= sh.nkv
            cls[(s_, j)] = 0 if not live else (1 if full else 3)
    return cls


def classify(words):
    live = np.any(words != 0xFC00FC00)
    nonzero = np.any((words & 0x7FFF7FFF) != 0)
    return 0 if not live else (3 if nonzero else 1)


def blocks_per_wave(nA, nB, hasA):
    """Largest number of blocks any wavefront of the pair computes."""
    wB = assignment(nA, nB, hasA)
    worst = 0
    for w in range(NW):
        onB = w < wB
        wT = wB if onB else NW - wB
        iT = w if onB else NW - 1 - w
        nT = nB if onB else nA
        worst = max(worst, (nT - iT + wT - 1) // wT if nT > iT else 0)
    return worst


def assignment(nA, nB, hasA, plant=None):
    wB = NW
    if hasA:
        if nA + nB == 0:
            wB = NW // 2
        else:
            wB = min(max((NW * nB + (nA + nB) // 2) // (nA + nB), 1), NW - 1)
    if plant == "wb_off_by_one" and hasA and nA > 0:
        wB = min(wB + 1, NW)
    return wB


def emulate_pair(sh: Shape, heads=None, batches=None, plant=None):
    """Run the checks for every workgroup of the given heads / batches
    (default: the first and the last). Returns a summary dict."""
    nt = (sh.nq + 31) // 32
    nk = (sh.nkv + TK - 1) // TK
    if nk > MAXK:
        raise ValueError("n_kv > 512 is not this kernel's")
    np_ = (nt + 1) // 2
    heads = heads if heads is not None else sorted({0, sh.hq - 1})
    batches = batches if batches is not None else sorted({0, sh.b - 1})
    buf = sh.mask_buffer() if sh.mode != "implicit" else None
    n_blocks = 0
    for bb in batches:
        for h in heads:
            hk = h // (sh.hq // sh.hkv)
            bkv = bb // (sh.b // sh.bk)
            stored = np.zeros((sh.nq, D), dtype=np.int32)
            for p in range(np_):
                n_blocks += _emulate_wg(sh, p, h, bb, hk, bkv, nt, nk, buf, stored, plant)
            _check(stored == 1, f"output elements stored {stored.min()}..{stored.max()} times (head {h}, batch {bb})")
    return {"blocks": n_blocks}


def _emulate_wg(sh, p, h, bb, hk, bkv, nt, nk, buf, stored, plant):
    tA, tB = p, nt - 1 - p
    hasA = tA < tB
    plane_off = sh.m_mis + (h % sh.hm) * sh.m_nb2 + (bb % sh.bm) * sh.m_nb3
    kb = hk * sh.k_nb2 + bkv * sh.k_nb3   # K and V share the cache layout

    # Q loads (all 512 threads)
    QCH = 16 if sh.q_f16 else 32
    QPT = 2 * 32 * QCH // 512
    for t in range(512):
        for u in range(QPT):
            i = t + 512 * u
            s, r, cch = i // (32 * QCH), (i // QCH) % 32, i % QCH
            row = min(32 * (tB if s else tA) + r, sh.nq - 1)
            a = row * sh.q_nb1 + h * sh.q_nb2 + bb * sh.q_nb3 + cch * 16
            rs = row * sh.q_nb1 + h * sh.q_nb2 + bb * sh.q_nb3
            _check(rs <= a and a + 16 <= rs + D * sh.qe and a + 16 <= sh.q_bytes(), "Q load outside its row")
            # rotary position of the row (F32 Q): positions[b][row], b n_q + row < B n_q
            _check(0 <= bb * sh.nq + row < sh.b * sh.nq, "rotary position read outside the positions")

    # classes
    cls = {}
    if sh.mode == "tensor":
        for w in range(NW):
            jB, jA = w, MAXK - 1 - w
            candB, candA = jB < nk, hasA and jA < nk
            cB = classify_kernel(sh, buf, plane_off, tB, jB if candB else 0, plant)
            cA = classify_kernel(sh, buf, plane_off, tA, jA if candA else 0, plant)
            if candB:
                cls[(1, jB)] = cB
            if candA:
                cls[(0, jA)] = cA
        # the kernel's classes equal the ones the entries give
        for (s_, j), c in cls.items():
            T = tB if s_ else tA
            rows = range(32 * T, min(32 * T + 32, sh.nq))
            vals = [int(sh.mask[bb % sh.bm, h % sh.hm, r, k]) for r in rows for k in range(TK * j, TK * j + TK)
                    if k < sh.nkv]
            live = any(v != NEG_INF for v in vals)
            zero = all(v in (0, 0x8000) for v in vals) and TK * j + TK <= sh.nkv
            want = 0 if not live else (1 if zero else 3)
            _check(c == want, f"class of ({T}, {j}): {c}, entries give {want}")
    elif sh.mode == "intervals":
        key = (bb % sh.bm, h % sh.hm)
        if key not in _TABLES.get(id(sh), {}):
            _TABLES.setdefault(id(sh), {})[key] = interval_table(sh, bb, h)
        tab = _TABLES[id(sh)][key]
        cls = classify_intervals(sh, tab, tA, tB, hasA, nk, plant)
        for (s_, j), c in cls.items():
            T = tB if s_ else tA
            rows = range(32 * T, min(32 * T + 32, sh.nq))
            vals = [int(sh.mask[bb % sh.bm, h % sh.hm, r, k]) for r in rows for k in range(TK * j, TK * j + TK)
                    if k < sh.nkv]
            live = any(v != NEG_INF for v in vals)
            zero = all(v in (0, 0x8000) for v in vals) and TK * j + TK <= sh.nkv
            want = 0 if not live else (1 if zero else 3)
            # sound for any mask: every block with a live entry computed, the
            # mask skipped only where every entry is 0
            _check(not (want and not c), f"block ({T}, {j}) with live entries classed dead")
            _check(not (c == 1 and want != 1), f"block ({T}, {j}) classed all-zero, entries give {want}")
            # exact when the tile's rows are intervals (or empty)
            if all(tab[r][0] != -2 for r in rows):
                _check(c == want, f"class of ({T}, {j}) from intervals: {c}, entries give {want}")
    else:
        for j in range(nk):
            cls[(1, j)] = cls_formula(sh, tB, j)
            if hasA:
                cls[(0, j)] = cls_formula(sh, tA, j)
    liveB = [j for j in range(nk) if cls.get((1, j), 0)]
    liveA = [j for j in range(nk) if hasA and cls.get((0, j), 0)]
    nA, nB = len(liveA), len(liveB)
    wB = assignment(nA, nB, hasA, plant)

    # blocks per wavefront
    computed = {}
    for w in range(NW):
        onB = w < wB
        wT = wB if onB else NW - wB
        iT = w if onB else NW - 1 - w
        live = liveB if onB else liveA
        nT = len(live)
        nblk = (nT - iT + wT - 1) // wT if nT > iT else 0
        T = tB if onB else tA
        for k in range(nblk):
            j = live[iT + k * wT]
            key = (T, j)
            computed[key] = computed.get(key, 0) + 1
    if sh.mode != "implicit":
        ent = lambda row, pos: sh.mask[bb % sh.bm, h % sh.hm, row, pos]
        for (T, j) in computed:
            if cls[(1 if T == tB else 0, j)] == 3:
                rows = range(32 * T, min(32 * T + 32, sh.nq))
                if sh.mode == "intervals" and all(tab[r][0] != -2 for r in rows):
                    # words from the intervals; rows past n_q are not stored
                    words = mask_words_interval(sh, tab, T, j, plant)
                    want = mask_words_expected(sh, ent, T, j)
                    real = np.array([32 * T + (ln & 31) < sh.nq for ln in range(64)])
                    # +0 and -0 both read as zero (the tensor may hold either)
                    _check(((words[real] & 0x7FFF7FFF) == (want[real] & 0x7FFF7FFF)).all(),
                           f"interval words of block ({T}, {j}) differ from the entries")
                else:
                    words = mask_words_kernel(sh, buf, plane_off, T, j, plant)
                    _check(words == mask_words_expected(sh, ent, T, j),
                           f"mask words of block ({T}, {j}) differ from the entries")
    want = {(tB, j) for j in liveB} | {(tA, j) for j in liveA}
    _check(set(computed) == want and all(v == 1 for v in computed.values()),
           f"blocks computed {sorted(computed.items())} != live {sorted(want)}")

    # K, then V copies: every used tile, wavefront w issues parts w and w + 8
    # into the same LDS area; then the operand reads of each computed block
    # (K: 16-byte A-operand reads, V^T: transposed 8-byte reads) must find the
    # global chunk they need
    used = sorted(set(liveA) | set(liveB))
    rl = LANES >> 4
    am, ahb, ab = (LANES & 31) >> 3, ((LANES & 31) >> 2) & 1, LANES & 3
    krow = np.where(ahb != 0, 16 + ((am + 2) & 3) * 4 + ab, 4 * am + ab)
    hh = LANES >> 5
    vq = (LANES & 15) >> 2
    clo = 2 * ((LANES & 31) >> 4) + ((LANES & 3) >> 1)
    for role in ("k", "v"):
        swz = swz_k if role == "k" else swz_v
        written = np.zeros(MAXK * VT, dtype=np.int32)
        src = np.full(MAXK * VT // 16, -1, dtype=np.int64)   # global chunk address landing in each LDS chunk
        for j in used:
            kv0 = TK * j
            for w in range(NW):
                for gg in range(2):
                    g = w + NW * gg
                    r = 4 * g + rl
                    col = ((LANES & 15) ^ swz(r)) * 16
                    dst = j * VT + 4 * g * ROW
                    if kv0 + TK <= sh.nkv and plant != "v_clamp_always_full":
                        kv = kv0 + r
                        ga = kb + kv0 * sh.k_nb1 + r * sh.k_nb1 + col
                    else:
                        kv = np.minimum(kv0 + r, sh.nkv - 1) if plant != "v_no_row_clamp" else kv0 + r
                        ga = kb + kv * sh.k_nb1 + col
                    _check(kv < sh.nkv, f"{role} copy reads row {kv.max()} >= n_kv {sh.nkv}")
                    rs = kb + kv * sh.k_nb1
                    _check((ga >= rs) & (ga + 16 <= rs + ROW) & (ga + 16 <= sh.kv_bytes()), f"{role} copy outside its row")
                    l = dst + 16 * LANES
                    _check((l >= 0) & (l + 16 <= MAXK * VT), f"{role} copy lands outside the LDS area")
                    for x in range(16):
                        np.add.at(written, l + x, 1)
                    src[l // 16] = ga
        for j in used:
            seg = written[j * VT:(j + 1) * VT]
            _check(seg == 1, f"{role} tile {j}: bytes written {seg.min()}..{seg.max()} times")
        for (T, j) in computed:
            if role == "k":
                kx = hh ^ swz_k(krow)
                for ks in range(KS):
                    for kvb in range(2):
                        addr = j * VT + krow * ROW + ((2 * ks) ^ kx) * 16 + 32 * kvb * ROW
                        _check((addr >= j * VT) & (addr + 16 <= (j + 1) * VT), "K read outside its tile")
                        kvr = np.minimum(TK * j + 32 * kvb + krow, sh.nkv - 1)
                        want = kb + kvr * sh.k_nb1 + (2 * ks + hh) * 16
                        _check(src[addr // 16] == want, "K operand read finds another row or chunk than it needs")
            else:
                for pc in range(4):
                    kvb, cc = pc >> 1, pc & 1
                    for db in range(DB):
                        for hi in range(2):
                            row_in_tile = np.where(hh != 0, 24 - 8 * cc, 8 * cc) + vq + 32 * kvb + 4 * hi
                            vaddr = j * VT + row_in_tile * ROW + ((4 * db + clo) ^ swz_v(vq)) * 16 + (LANES & 1) * 8
                            _check((vaddr >= j * VT) & (vaddr + 8 <= (j + 1) * VT), "V^T read outside its tile")
                            _check(written[vaddr] == 1, "V^T read of an unwritten byte")
                            kvr = np.minimum(TK * j + row_in_tile, sh.nkv - 1)
                            want = kb + kvr * sh.k_nb1 + (4 * db + clo) * 16
                            _check(src[vaddr // 16] == want, "V^T read finds another row or chunk than it needs")

    # merge and store: a wavefront of a tile with others publishes its 16
    # groups (16-byte chunk (w, q, lane) at byte 16 (1024 w + 64 q + lane) of
    # the V area); tile T's wavefronts each take groups iT, iT + wT, ... and
    # read group q of every wavefront of the tile; a lone wavefront stores its
    # own 16 groups
    published = set()
    for w in range(NW):
        onB = w < wB
        wT = wB if onB else NW - wB
        if wT > 1:
            for q in range(16):
                off = 16 * (1024 * w + 64 * q + LANES)
                _check((off >= 0) & (off + 16 <= MAXK * VT), "published chunk outside the V area")
                published.add((w, q))
    for w in range(NW):
        onB = w < wB
        if not onB and not hasA:
            continue
        wT = wB if onB else NW - wB
        iT = w if onB else NW - 1 - w
        T = tB if onB else tA
        g0 = 0 if onB else wB
        for q in range(iT, 16, wT):
            if wT > 1:
                for gi in range(NW):
                    g = g0 + min(gi, wT - 1)
                    _check((g, q) in published and ((g < wB) == onB), "merge reads a group nobody of the tile published")
            dbq, a4 = q >> 2, q & 3
            for lane in range(64):
                row = 32 * T + (lane & 31)
                if row < sh.nq:
                    d0 = 32 * dbq + 8 * a4 + 4 * (lane >> 5)
                    stored[row, d0:d0 + 4] += 1
    return len(computed)
