"""Host checks of the mask-tensor path of the hd 64 pipelined kernel
(fa_prefill_pp.hip), run on the CPU before any GPU run:

  * the pre-pass (mask_rows_kernel) restated chunk by chunk
    (dma_emul.mask_row_interval) classifies every row as the definition
    says: (lo, hi) for a row that is +-0 on [lo, hi] and -inf elsewhere,
    (n, -1) for a row of -inf only, (-2, -2) for anything else (finite
    non-zero entries, -inf holes inside), at every row alignment the API
    accepts (2-byte), reading only chunks that hold a byte of the row;
  * the realtime encoder's sliding-window mask (src/voxtral.cpp:2179-2190,
    window 750) gives exactly the implicit window's intervals, so the mask
    tensor and the implicit mask walk the same blocks with the same bounds;
  * the block ranges the kernel derives from the table cover exactly the
    live blocks of each workgroup's rows, and the copy schedule over them
    stays in bounds with its waits (dma_emul.emulate_pp)."""
import numpy as np
import pytest

from dma_emul import NEG_INF_F16, Shape, emulate_pp, mask_row_interval, pp_block_range, pp_block_range_table

NEG0 = 0x8000
ONE = 0x3C00


def classify(row):
    """The definition, over the whole row at once."""
    row = np.asarray(row, dtype=np.uint16)
    fin = row != NEG_INF_F16
    if np.any((row[fin] & 0x7FFF) != 0):
        return (-2, -2)
    idx = np.flatnonzero(fin)
    if idx.size == 0:
        return (len(row), -1)
    lo, hi = int(idx[0]), int(idx[-1])
    return (lo, hi) if fin[lo:hi + 1].all() else (-2, -2)


def rows_of_every_kind(n, rng):
    out = []
    z = np.zeros(n, np.uint16)
    out.append(z.copy())                                   # all live
    out.append(np.full(n, NEG_INF_F16, np.uint16))         # none live
    for _ in range(6):                                     # one interval
        lo = int(rng.integers(0, n))
        hi = int(rng.integers(lo, n))
        r = np.full(n, NEG_INF_F16, np.uint16)
        r[lo:hi + 1] = 0
        if hi > lo:
            r[int(rng.integers(lo, hi + 1))] = NEG0      # -0 is live, zero
        out.append(r)
        if hi - lo >= 2:                                   # a hole inside
            h = r.copy()
            h[int(rng.integers(lo + 1, hi))] = NEG_INF_F16
            out.append(h)
        f = r.copy()                                       # a finite non-zero entry
        f[int(rng.integers(lo, hi + 1))] = ONE
        out.append(f)
    e = np.full(n, NEG_INF_F16, np.uint16)                 # live only at an end
    e[-1] = 0
    out.append(e)
    s = np.full(n, NEG_INF_F16, np.uint16)
    s[0] = 0
    out.append(s)
    return out


@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 31, 32, 33, 100, 257, 1500])
def test_pre_pass_classifies_rows(n):
    rng = np.random.default_rng(n)
    for row in rows_of_every_kind(n, rng):
        want = classify(row)
        for mis in range(0, 16, 2):
            assert mask_row_interval(row, mis) == want, (n, mis, row)


def test_classification_separates_holes_and_values():
    """The cases the fast path must not take: a hole (lo and hi alone would
    call it an interval) and a finite non-zero entry."""
    r = np.full(64, NEG_INF_F16, np.uint16)
    r[10:20] = 0
    assert mask_row_interval(r, 6) == (10, 19)
    r[15] = NEG_INF_F16
    assert mask_row_interval(r, 6) == (-2, -2)
    r[15] = 0
    r[12] = 0x3800   # 0.5
    assert mask_row_interval(r, 6) == (-2, -2)


def window_mask(n, w):
    """src/voxtral.cpp:2179-2190: row q attends max(0, q - (w - 1)) <= kv <= q."""
    q = np.arange(n)[:, None]
    kv = np.arange(n)[None, :]
    allow = (kv <= q) & (kv >= np.maximum(0, q - (w - 1)))
    return np.where(allow, 0, NEG_INF_F16).astype(np.uint16)


def test_realtime_window_gives_the_implicit_intervals():
    n, w = 1500, 750
    m = window_mask(n, w)
    # the chunk walk (mask_row_interval) is checked against classify above;
    # every 97th row takes it here too (3000-byte rows: 8-byte misalignment
    # on odd rows)
    table = [classify(m[q]) for q in range(n)]
    for q in range(0, n, 97):
        assert mask_row_interval(m[q], (q * 2 * n) % 16) == table[q]
    assert table == [(max(0, q - w + 1), q) for q in range(n)]
    sh = Shape(n, n, 32, 32)
    for qg in range((n + 127) // 128):
        assert pp_block_range_table(sh, qg, table) == pp_block_range(sh, qg, 128, w, 0)


def _live_blocks(table, rows, nkv):
    live = set()
    for r in rows:
        lo, hi = table[r]
        if lo == -2:
            return set(range((nkv + 31) // 32))
        live.update(range(lo // 32, hi // 32 + 1) if lo <= hi else ())
    return live


def _tables(nq, nkv, rng):
    yield "window", [classify(r) for r in window_mask(max(nq, nkv), 100)[:nq, :nkv]]
    causal = [(0, min(q, nkv - 1)) for q in range(nq)]
    yield "causal", causal
    ivl = []
    for q in range(nq):
        k = int(rng.integers(0, 4))
        if k == 0:
            ivl.append((nkv, -1))
        else:
            lo = int(rng.integers(0, nkv))
            ivl.append((lo, int(rng.integers(lo, nkv))))
    yield "random", ivl
    slow = list(ivl)
    slow[nq // 2] = (-2, -2)
    yield "slow", slow
    yield "empty", [(nkv, -1)] * nq


@pytest.mark.parametrize("nq,nkv", [(1500, 1500), (439, 439), (129, 64), (300, 1000), (64, 32), (200, 97)])
def test_table_ranges_cover_live_blocks_and_copies_stay_in_bounds(nq, nkv):
    rng = np.random.default_rng(nq * 7 + nkv)
    sh = Shape(nq, nkv, 2, 2)
    for name, table in _tables(nq, nkv, rng):
        for qg in range((nq + 127) // 128):
            blo, nb = pp_block_range_table(sh, qg, table)
            live = _live_blocks(table, range(qg * 128, min(qg * 128 + 128, nq)), nkv)
            assert set(range(blo, blo + nb)) == live, (name, qg, blo, nb)
        emulate_pp(sh, table=table)


@pytest.mark.parametrize("stage_blocks,nrows", [(0, 1500), (375, 1500), (235, 1), (1, 17), (55, 439)])
def test_prep_launch_partition(stage_blocks, nrows):
    """prep_kernel (the mask pre-pass and F32 staging in one launch of
    256-thread blocks): blocks [0, nmb) take four mask rows each, one per
    wavefront, bx * 4 + tid / 64, rows past nrows reading row nrows - 1 and
    storing nothing; blocks [nmb, nmb + 2 sb) stage tensor (bx - nmb) / sb,
    block (bx - nmb) % sb. mask_rows_kernel is the first part alone. Every
    staging block of both tensors and every mask row is covered exactly
    once."""
    sb = stage_blocks
    nmb = (nrows + 3) // 4
    nb = nmb + 2 * sb
    staged, rows = [], []
    for bx in range(nb):
        if bx >= nmb:
            sx = bx - nmb
            staged.append((sx // sb, sx % sb))
            continue
        for tid in range(0, 256, 64):               # lane 0 of each row's wavefront stores
            w = bx * 4 + tid // 64
            wr = min(w, nrows - 1)
            assert 0 <= wr < nrows
            if w < nrows:
                rows.append(w)
    assert sorted(staged) == [(t, b) for t in range(2) for b in range(sb)]
    assert sorted(rows) == list(range(nrows))
