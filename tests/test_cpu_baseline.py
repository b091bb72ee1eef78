"""The timed CPU baseline (oracle/fa_cpu_simd.c: ggml's one-row algorithm
with its AVX2/F16C vector kernels) computes the same bits as the scalar
restatement in f16-accumulator mode (oracle/fa_oracle.c), which the other
oracle tests pin: the dot products use the same 32 partial sums reduced in
the same pairwise order, Q and the V accumulator round to f16 the same way,
and both call libm's expf. Runs without a GPU."""
import numpy as np
import pytest

import cases
from oracle import oracle

CASES = [
    lambda: cases.decode_case(300, hq=32, hkv=8, hd=128, seed=71),
    lambda: cases.decode_case(150, hq=4, hkv=1, hd=64, seed=72, window=40),
    lambda: cases.decode_case(90, hq=8, hkv=2, hd=128, seed=73, batch=3),
    lambda: cases.decode_case(70, hq=8, hkv=8, hd=64, seed=74, q_f16=True),
    lambda: cases.encoder_case(61, 3, 64, seed=75),
    lambda: cases.encoder_case(50, 2, 64, seed=76, window=20),
    lambda: cases.prefill_case(33, hq=8, hkv=2, seed=77),
    lambda: cases.prefill_case(20, hq=4, hkv=1, seed=78, kv_offset=45, capacity=80),
    lambda: cases.batched_case(4, hq=8, hkv=2, capacity=96, lo=5, hi=96, seed=79),
]


def _simd(c, threads):
    v = c.oracle_view
    return oracle.fa_cpu_simd(v("q"), v("k"), v("v"), v("mask"), c.scale, threads=threads)


@pytest.mark.parametrize("make", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_simd_baseline_equals_scalar_restatement(make):
    c = make()
    want = cases.oracle_ggml(c, vkq_f16=True)
    for threads in (1, 5):
        got = _simd(c, threads)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_simd_baseline_rejects_f32_kv():
    c = cases.decode_case(40, hq=8, hkv=2, hd=128, seed=80, kv_f32=True)
    with pytest.raises(ValueError):
        _simd(c, 1)


def test_host_thread_counts():
    assert 1 <= oracle.default_threads() <= min(oracle.host_threads(), 16)
