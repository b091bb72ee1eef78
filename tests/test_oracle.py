"""Pins the CPU oracle (oracle/fa_oracle.c) without a GPU.

The op's reference arithmetic lives in ggml (ggml-org/ggml@5cecdad, fetched
by the reference's CMakeLists.txt:29-39, absent here), and the reference
holds no golden vectors for it. The oracle is therefore pinned by:
  * a library routine: torch's scaled_dot_product_attention in float64 on
    the same bytes (tests/refmath.py), for every layout voxtral.cpp builds;
  * closed forms and special cases (n_kv = 1, q = 0, a dominant score,
    fully masked rows, distinct-constant KV heads);
  * invariants (KV permutation, constant mask offset, linearity in V,
    contiguous vs permuted views);
  * planted mistakes: each ORACLE_MUT_* flag must fail one of the checks;
  * the committed fixtures under tests/golden/.
"""
import math

import numpy as np
import pytest

import cases
import refmath
from oracle import oracle

ATOL, RTOL = 2e-3, 1e-2


def rel_err(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))


# --- binary16 conversions against numpy's float16 (a library routine) -------

def test_f16_to_f32_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        rng.standard_normal(50000).astype(np.float32) * np.float32(1e-5),   # subnormal range
        rng.standard_normal(20000).astype(np.float32) * np.float32(4e4),    # overflow edge
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 5.96e-8, 2.98e-8, 2.99e-8,
                  6.1035e-5, 6.1e-5, np.inf, -np.inf], dtype=np.float32),
    ])
    # exact ties: f16 values plus half an ulp
    h = rng.integers(0, 0x7BFF, 5000).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    up = (h + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    x = np.concatenate([x, (f + (up - f) / 2).astype(np.float32)])
    got = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    nanbits = oracle.f32_to_f16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(nanbits.view(np.float16)).all()


# --- the f64 oracle against torch SDPA (float64) on voxtral's layouts --------

SMALL_CASES = [
    lambda: cases.decode_case(37, hq=8, hkv=2, hd=128, seed=1),
    lambda: cases.decode_case(200, hq=32, hkv=8, hd=128, capacity=260, seed=2),
    lambda: cases.decode_case(150, hq=4, hkv=1, hd=64, seed=3, window=40),
    lambda: cases.decode_case(90, hq=8, hkv=2, hd=128, seed=4, batch=3),
    lambda: cases.decode_case(70, hq=8, hkv=8, hd=64, seed=5, q_f16=True),
    lambda: cases.encoder_case(61, 3, 64, seed=6),
    lambda: cases.encoder_case(50, 2, 64, seed=7, window=20),
    lambda: cases.prefill_case(33, hq=8, hkv=2, seed=8),
    lambda: cases.prefill_case(20, hq=4, hkv=1, seed=9, kv_offset=45, capacity=80),
    lambda: cases.prefill_case(25, hq=4, hkv=2, seed=10, causal=False),
    lambda: cases.batched_case(4, hq=8, hkv=2, capacity=96, lo=5, hi=96, seed=11),
    # F32 K/V: the reference's own cache type and encoder K/V (Q stays F32)
    lambda: cases.decode_case(120, hq=8, hkv=2, hd=128, seed=12, kv_f32=True),
    lambda: cases.encoder_case(45, 2, 64, seed=13, kv_f32=True),
    lambda: cases.prefill_case(30, hq=4, hkv=1, seed=14, kv_offset=9, kv_f32=True),
]


@pytest.mark.parametrize("make", SMALL_CASES, ids=[f"c{i}" for i in range(len(SMALL_CASES))])
def test_f64_oracle_matches_torch_sdpa(make):
    c = make()
    want, live = refmath.sdpa_f64(c)
    got = cases.oracle_f64(c)
    assert np.allclose(got[live], want[live], rtol=1e-10, atol=1e-12)
    assert (got[~live] == 0).all()   # fully masked rows give zeros (ggml: S == 0 -> 0)


@pytest.mark.parametrize("make", SMALL_CASES, ids=[f"c{i}" for i in range(len(SMALL_CASES))])
def test_ggml_restatement_within_tolerance_of_exact(make):
    """fp32 accumulation (the bar's "fp32 accumulate") is within the parity tolerance."""
    c = make()
    exact = cases.oracle_f64(c)
    got = cases.oracle_ggml(c, vkq_f16=False)
    assert float(np.abs(got - exact).max()) <= ATOL
    assert rel_err(got, exact) <= RTOL


@pytest.mark.parametrize("make", SMALL_CASES, ids=[f"c{i}" for i in range(len(SMALL_CASES))])
def test_ggml_f16_accumulator_spread(make):
    """The one-row kernel's f16 V accumulator rounds every update to 11 bits:
    its spread from exact is about one f16 ulp of the output (2^-11 near 1,
    up to ~3e-3 here), above the 2e-3 max-abs bar, and far below 1e-2
    relative. This is why parity is stated against fp32 accumulation and the
    f16 mode is only a bracket."""
    c = make()
    exact = cases.oracle_f64(c)
    got = cases.oracle_ggml(c, vkq_f16=True)
    assert float(np.abs(got - exact).max()) <= 5e-3
    assert rel_err(got, exact) <= RTOL


def test_thread_count_does_not_change_bits():
    c = cases.prefill_case(40, hq=8, hkv=2, seed=12)
    a = cases.oracle_ggml(c, threads=1)
    b = cases.oracle_ggml(c, threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# --- special cases with closed forms ------------------------------------------

def _vals(c, role, shape):
    return c.bufs[role].view(np.float16).astype(np.float64).reshape(shape)


def test_single_position_returns_v():
    c = cases.decode_case(1, hq=8, hkv=2, hd=128, seed=20)
    v = _vals(c, "v", (1, 2, 128))
    for fn in (cases.oracle_f64, cases.oracle_ggml):
        out = fn(c)
        for h in range(8):
            assert np.array_equal(out[0, 0, h].astype(np.float64), v[0, h // 4])


def test_zero_query_gives_mean_of_v():
    c = cases.decode_case(57, hq=4, hkv=2, hd=64, seed=21)
    c.bufs["q"][...] = 0
    v = _vals(c, "v", (57, 2, 64))
    out = cases.oracle_ggml(c)
    for h in range(4):
        assert np.allclose(out[0, 0, h], v[:, h // 2].mean(axis=0), atol=1e-5)


def test_dominant_score_selects_one_row():
    c = cases.decode_case(40, hq=2, hkv=1, hd=64, seed=22)
    k = c.bufs["k"].view(np.float16).reshape(40, 1, 64)
    k[...] = np.float16(0.0)
    k[17, 0, :] = np.float16(4.0)
    c.bufs["q"][...] = 4.0            # score 4*4*64/8 = 128 at position 17, 0 elsewhere
    v = _vals(c, "v", (40, 1, 64))
    out = cases.oracle_ggml(c)
    assert np.allclose(out[0, 0, 0], v[17, 0], atol=1e-6)


def test_gqa_mapping_with_constant_heads():
    """KV head j holds the constant j + 1 in V: query head h must read h / (Hq/Hkv)."""
    c = cases.decode_case(30, hq=8, hkv=4, hd=128, seed=23)
    v = c.bufs["v"].view(np.float16).reshape(30, 4, 128)
    for j in range(4):
        v[:, j, :] = np.float16(j + 1)
    out = cases.oracle_ggml(c)
    for h in range(8):
        assert np.allclose(out[0, 0, h], h // 2 + 1, atol=1e-6)


def test_fully_masked_row_is_zero_and_others_unaffected():
    c = cases.prefill_case(12, hq=2, hkv=1, seed=24)
    m = c.bufs["mask"].reshape(12, 12)
    m[4, :] = cases.NEG_INF_F16
    out = cases.oracle_ggml(c)
    assert (out[0, 4] == 0).all()
    want, _ = refmath.sdpa_f64(c)
    keep = [i for i in range(12) if i != 4]
    assert np.abs(out[0, keep] - want[0, keep]).max() <= ATOL


def test_masked_positions_are_skipped_not_added():
    """-inf positions vanish even when every live score is very negative."""
    c = cases.decode_case(64, hq=2, hkv=1, hd=64, seed=25, window=8)
    c.bufs["q"][...] = -30.0
    c.bufs["k"].view(np.float16)[...] = np.float16(1.0)
    v = _vals(c, "v", (64, 1, 64))
    out = cases.oracle_ggml(c)
    assert np.allclose(out[0, 0, 0], v[-8:, 0].mean(axis=0), atol=1e-5)


# --- invariants ----------------------------------------------------------------

def test_kv_permutation_invariance():
    c = cases.decode_case(80, hq=4, hkv=1, hd=128, seed=26, window=50)
    base = cases.oracle_f64(c)
    perm = np.random.default_rng(26).permutation(80)
    for name in ("k", "v"):
        c.bufs[name] = c.bufs[name].reshape(80, 1, 128)[perm].reshape(-1).copy()
    c.bufs["mask"] = c.bufs["mask"].reshape(1, 1, 80)[..., perm].copy()
    assert np.allclose(cases.oracle_f64(c), base, atol=1e-12)


def test_constant_mask_offset_invariance():
    c = cases.prefill_case(16, hq=2, hkv=1, seed=27)
    base = cases.oracle_f64(c)
    m = c.bufs["mask"]
    c.bufs["mask"] = np.where(m == cases.NEG_INF_F16, m, cases.f16_bits(np.float32([3.0]))[0]).astype(np.uint16)
    assert np.allclose(cases.oracle_f64(c), base, atol=1e-12)


def test_linearity_in_v():
    c = cases.decode_case(50, hq=2, hkv=1, hd=64, seed=28)
    v = c.bufs["v"].view(np.float16)
    a = cases.oracle_f64(c)
    v[...] = (v.astype(np.float32) * 2).astype(np.float16)   # exact in f16
    assert np.allclose(cases.oracle_f64(c), 2 * a, atol=1e-12)


def test_strided_and_contiguous_views_agree():
    """The encoder's permuted view [hd, seq, heads] of a [seq][heads][hd] buffer
    gives the same result as head-major contiguous copies."""
    c = cases.encoder_case(30, 3, 64, seed=29)
    a = cases.oracle_f64(c)
    for role in ("q", "k", "v"):
        b, t, ne, nb, off = c.views[role]
        arr = c.bufs[b]
        elt = nb[0]
        dt = np.float32 if t == oracle.F32 else np.uint16
        hm = arr.view(dt).reshape(30, 3, 64).transpose(1, 0, 2).copy()   # [heads][seq][hd]
        c.bufs[b] = hm
        c.views[role] = (b, t, ne, (elt, 64 * elt, 30 * 64 * elt, 3 * 30 * 64 * elt), 0)
    assert np.array_equal(cases.oracle_f64(c), a)


# --- planted mistakes must be caught -------------------------------------------

@pytest.mark.parametrize("flag", [oracle.MUT_GQA_MOD, oracle.MUT_NO_MASK, oracle.MUT_NO_SCALE,
                                  oracle.MUT_V_SHIFT, oracle.MUT_NO_MAXSUB])
def test_planted_mistakes_fail_the_check(flag):
    c = cases.prefill_case(24, hq=8, hkv=2, seed=30, kv_offset=8)
    want, _ = refmath.sdpa_f64(c)
    ok = cases.oracle_ggml(c)
    assert float(np.abs(ok - want).max()) <= ATOL
    bad = cases.oracle_ggml(c, flags=flag)
    assert float(np.abs(bad - want).max()) > 10 * ATOL


def test_f32_kv_keeps_q_unrounded():
    """With F32 K ggml keeps Q in F32 (K's dot type): the restatement's and
    the f64 reference's results then differ from the Q-rounded reference by
    more than they differ from each other."""
    c = cases.decode_case(64, hq=4, hkv=1, hd=128, seed=15, kv_f32=True, q_sigma=3.0)
    exact = cases.oracle_f64(c)
    rounded = cases.oracle_f64(c, q_f16=True)
    got = cases.oracle_ggml(c, vkq_f16=False)
    assert float(np.abs(got - exact).max()) < 1e-5
    assert float(np.abs(rounded - exact).max()) > 10 * float(np.abs(got - exact).max())


@pytest.mark.parametrize("max_bias,softcap", [(8.0, 0.0), (0.0, 30.0)])
def test_alibi_and_softcap_are_rejected(max_bias, softcap):
    """voxtral passes 0 for both (src/voxtral.cpp:1611, :1802); the oracle
    restates neither and reports them as a contract violation."""
    c = cases.decode_case(16, hq=4, hkv=1, hd=64, seed=33)
    with pytest.raises(ValueError):
        oracle.fa_ggml(c.oracle_view("q"), c.oracle_view("k"), c.oracle_view("v"), None, c.scale,
                       max_bias=max_bias, logit_softcap=softcap)
    with pytest.raises(ValueError):
        oracle.fa_f64(c.oracle_view("q"), c.oracle_view("k"), c.oracle_view("v"), None, c.scale,
                      max_bias=max_bias, logit_softcap=softcap)


def test_contract_violation_is_reported():
    c = cases.decode_case(10, hq=6, hkv=4, hd=64, seed=31)   # 6 % 4 != 0
    with pytest.raises(ValueError):
        cases.oracle_ggml(c)


def test_scale_follows_float32_param():
    """ggml stores scale as a float op param: 1/sqrt(128) as float32."""
    c = cases.decode_case(5, hq=2, hkv=1, hd=128, seed=32)
    assert c.scale == float(np.float32(1.0 / math.sqrt(128)))
