"""CPU checks of the short masked prefill kernel's addressing and work
assignment (tests/pair_emul.py restates voxtral.cpp_amd/csrc/fa_prefill_pair.hip):
reads inside their rows and granules, copies inside the V area, mask words
equal to the entries, every live block computed once, every output element
stored once."""
import numpy as np
import pytest

from pair_emul import NEG_INF, Shape, Violation, emulate_pair


def _window_mask(nq, nkv, offset, window):
    i = np.arange(nq)[:, None]
    j = np.arange(nkv)[None, :]
    live = (j <= i + offset) & (j >= i + offset - window + 1)
    return np.where(live, 0, NEG_INF).astype(np.uint16)[None, None]


def _random_mask(nq, nkv, seed, hm=1, bm=1):
    rng = np.random.default_rng(seed)
    m = np.where(rng.random((bm, hm, nq, nkv)) < 0.6, NEG_INF, 0).astype(np.uint16)
    fin = rng.random((bm, hm, nq, nkv)) < 0.1
    m[fin] = np.float16(-1.5).view(np.uint16)
    m[..., 5, :] = NEG_INF                       # a fully masked row
    return m


SHAPES = [
    Shape(439, 439),                                        # voxtral's decoder prefill, 878-byte mask rows
    Shape(439, 439, mode="implicit"),
    Shape(439, 439, m_mis=2),
    Shape(439, 439, m_mis=14, q_f16=True),
    Shape(2, 2), Shape(31, 31), Shape(32, 32), Shape(33, 33), Shape(64, 64), Shape(65, 65, m_mis=6),
    Shape(512, 512), Shape(511, 511, mode="implicit"),
    Shape(100, 300, offset=200),                            # prefill against a filled cache
    Shape(100, 300, offset=200, mode="implicit"),
    Shape(300, 300, mode="implicit", window=100),
    Shape(300, 300, mode="implicit", window=1),
    Shape(200, 437, offset=237, mode="implicit", window=50),
    Shape(300, 300, mask=_window_mask(300, 300, 0, 100)),
    Shape(130, 257, mask=_random_mask(130, 257, 1)),
    Shape(96, 500, hq=4, hkv=2, b=3, bk=3, hm=2, bm=3, m_mis=4, mask=_random_mask(96, 500, 2, hm=2, bm=3)),
    Shape(77, 77, hq=8, hkv=1, b=2, bk=1, m_nb1=256),       # padded rows, GQA 8, kv batch broadcast
    # classes from the mask pre-pass's intervals (F32 K/V staged in the same launch)
    Shape(339, 439, offset=100, mode="intervals"),          # voxtral's decoder prefill after 100 cached rows
    Shape(439, 439, m_mis=2, mode="intervals"),
    Shape(300, 300, mode="intervals", mask=_window_mask(300, 300, 0, 100)),
    Shape(130, 257, mode="intervals", mask=_random_mask(130, 257, 3)),   # holes and finite values: fallback
    Shape(96, 500, hq=4, hkv=2, b=3, bk=3, hm=2, bm=3, m_mis=4, mode="intervals",
          mask=_random_mask(96, 500, 4, hm=2, bm=3)),
    Shape(65, 65, m_mis=6, mode="intervals"),
]


@pytest.mark.parametrize("sh", SHAPES, ids=lambda s: f"{s.mode}-{s.nq}x{s.nkv}-mis{s.m_mis}-w{s.window}")
def test_pair_addressing_and_assignment(sh):
    r = emulate_pair(sh)
    assert r["blocks"] > 0


def test_causal_439_one_block_per_wavefront():
    # 14 tiles of 32 rows: every pair holds 8 live blocks, one per wavefront
    from pair_emul import assignment, cls_formula
    sh = Shape(439, 439, mode="implicit")
    for p in range(7):
        tA, tB = p, 13 - p
        nA = sum(1 for j in range(7) if cls_formula(sh, tA, j))
        nB = sum(1 for j in range(7) if cls_formula(sh, tB, j))
        assert nA + nB == 8
        assert assignment(nA, nB, True) == nB


def test_at_most_two_blocks_per_wavefront():
    # up to 8 live KV tiles per query tile: no wavefront computes more than 2 blocks
    from pair_emul import blocks_per_wave
    for nA in range(9):
        for nB in range(9):
            assert blocks_per_wave(nA, nB, True) <= 2, (nA, nB)
        assert blocks_per_wave(0, nA, False) <= 1


@pytest.mark.parametrize("plant", ["no_chunk_clamp", "wb_off_by_one", "v_no_row_clamp"])
def test_pair_emulation_catches_planted_mistakes(plant):
    with pytest.raises(Violation):
        emulate_pair(Shape(439, 439), plant=plant)


@pytest.mark.parametrize("plant", ["holds_ignores_hi", "non_interval_dead", "interval_words_hi_open"])
def test_interval_classes_catch_planted_mistakes(plant):
    """The pre-pass route: a block counted as wholly covered by an interval
    that ends inside it, a non-interval row's blocks left dead, or mask words
    formed with an interval one entry too long each fail the check against
    the entries."""
    sh = Shape(339, 439, offset=100, mode="intervals") if plant != "non_interval_dead" else \
        Shape(130, 257, mode="intervals", mask=_random_mask(130, 257, 3))
    with pytest.raises(Violation):
        emulate_pair(sh, plant=plant)
