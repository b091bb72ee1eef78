"""CPU emulation of the LDS-DMA copy schedule of the hd 64 encoder kernel
(fa_prefill_pp.hip): global source ranges, LDS targets and the s_waitcnt
vmcnt accounting against the barriers, for every KV group and wavefront of
each shape (see tests/dma_emul.py). Runs without a GPU."""
import pytest

from dma_emul import Mem, Shape, Violation, emulate_pp, pp_copy

# the encoder configuration, every encoder length the GPU tests use, GQA,
# batches, empty KV groups (n_kv < 4 blocks), partial last blocks and wide
# row strides (a K/V view inside a larger cache)
SHAPES = [Shape(1500, 1500, 20, 20)] + [Shape(n, n, 4, 4) for n in (1, 2, 31, 32, 33, 64, 96, 128, 161, 300, 700)] + [
    Shape(1024, 1024, 3, 3), Shape(257, 257, 8, 2), Shape(200, 97, 4, 4, b=3, bk=3),
    Shape(129, 4097, 2, 2), Shape(64, 1500, 2, 1, k_nb1=(8 << 20) - 16, v_nb1=(8 << 20) - 16),
]


@pytest.mark.parametrize("sh", SHAPES, ids=lambda s: f"nq{s.nq}_nkv{s.nkv}_h{s.hq}x{s.hkv}_b{s.b}_nb{s.k_nb1}")
def test_pp_copies_and_waits_in_bounds(sh):
    emulate_pp(sh)


# implicit causal / window masks: every workgroup walks only its rows' live
# blocks (the realtime encoder's window 750, causal, offsets, windows of one
# block and less, rows with no live position)
WINDOWS = [(Shape(1500, 1500, 32, 32), 750, 0), (Shape(1500, 1500, 4, 4), 0, 0), (Shape(439, 439, 4, 4), 0, 0),
           (Shape(300, 1000, 2, 2), 100, 600), (Shape(200, 200, 2, 2), 1, 0), (Shape(257, 300, 2, 2), 31, 5),
           (Shape(129, 64, 2, 2), 0, -100), (Shape(100, 4097, 1, 1), 2048, 3997), (Shape(64, 32, 1, 1), 33, 0)]


@pytest.mark.parametrize("sh,window,offset", WINDOWS, ids=lambda v: str(v) if not isinstance(v, Shape) else f"nq{v.nq}_nkv{v.nkv}")
def test_pp_window_copies_and_waits_in_bounds(sh, window, offset):
    r = emulate_pp(sh, window=window, offset=offset)
    # the ranges cover exactly the live blocks of each workgroup's rows
    from dma_emul import pp_block_range
    for qg in range((sh.nq + 127) // 128):
        blo, nb = pp_block_range(sh, qg, 128, window, offset)
        rows = range(qg * 128, min(qg * 128 + 128, sh.nq))
        live = set()
        for i in rows:
            lo = i + offset - window + 1 if window > 0 else 0
            for j in range(max(lo, 0), min(i + offset + 1, sh.nkv)):
                live.add(j // 32)
        assert live == set(range(blo, blo + nb)) or (not live and nb == 0), (qg, blo, nb)


@pytest.mark.parametrize("plant", ["wait_late", "copy_early"])
def test_schedule_emulation_catches_planted_mistakes(plant):
    """A wait one block short, or a copy one block further ahead (into the
    slot of a block still to be read), is reported."""
    with pytest.raises(Violation):
        emulate_pp(Shape(1500, 1500, 20, 20), plant=plant)


def test_emulation_catches_planted_mistakes():
    """The checks fire: a block read with one copy too many still in flight,
    and a copy of the partial block without the row clamp."""
    m = Mem()
    for blk in (0, 1):
        for _ in range(8):
            m.issue(blk)
    m.wait(9)   # one of block 0's copies still outstanding
    assert not m.complete(0)
    m.wait(8)
    assert m.complete(0) and not m.complete(1)
    sh = Shape(100, 100, 1, 1)
    import dma_emul
    orig = dma_emul.np.minimum
    try:
        dma_emul.np.minimum = lambda a, b: a   # drop the clamp of rows past n_kv
        with pytest.raises(Violation):
            pp_copy(sh, 2, 4, 4, 0, 0, 3, 0, Mem())   # block 3 = rows 96..127 of 100
    finally:
        dma_emul.np.minimum = orig


# ---- the masked hd 128 prefill (fa_prefill.hip), shipped and reordered ----

from prefill_emul import emulate_prefill_masked  # noqa: E402

# decoder prefill 439 causal (the shape whose reordered variant faulted),
# prefills after cached rows, a single row group, n_kv past one step, a
# sliding window (workgroups whose live range starts past step 0) and rows
# with no live position
PREFILL_CASES = [
    dict(nq=439, nkv=439), dict(nq=100, nkv=439), dict(nq=64, nkv=8192), dict(nq=1, nkv=129),
    dict(nq=300, nkv=1000, mask_fn=lambda i, j: i + 700 - 200 < j <= i + 700),
    dict(nq=130, nkv=300, mask_fn=lambda i, j: i < 64 and j <= i),
]


@pytest.mark.parametrize("order", ["shipped", "copies_first"])
@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: f"nq{c['nq']}_nkv{c['nkv']}")
def test_masked_prefill_schedule(case, order):
    """Copies in bounds, no LDS access racing a copy in flight, every step's
    copies landed before its reads, no wavefront ending with a copy in
    flight: for the shipped order and for step 0's copies issued before the
    mask scan."""
    emulate_prefill_masked(order=order, **case)


@pytest.mark.parametrize("plant", ["issue_after_wait", "same_stage", "prefetch_at_end", "past_nkv"])
def test_masked_prefill_emulation_catches_planted_mistakes(plant):
    """A copy issued after the wait meant to cover it, a next step copied into
    the stage being read, a copy still in flight when the wavefront ends, a
    step past n_kv: each is reported."""
    with pytest.raises(Violation):
        emulate_prefill_masked(439, 439, order="shipped", plant=plant)
    if plant != "issue_after_wait":   # the reordered form issues step 0 before every wait
        with pytest.raises(Violation):
            emulate_prefill_masked(439, 439, order="copies_first", plant=plant)
