"""The oracle against the committed fixtures (tests/golden/, written by
tests/golden/make_golden.py from torch's float64 SDPA on the same bytes)."""
import numpy as np
import pytest

import cases
import golden_util

ATOL, RTOL = 2e-3, 1e-2


def test_fixtures_present():
    assert len(golden_util.names()) >= 8


@pytest.mark.parametrize("name", golden_util.names())
def test_f64_oracle_reproduces_fixture(name):
    c, want = golden_util.load(name)
    got = cases.oracle_f64(c)
    assert got.shape == want.shape
    assert np.allclose(got, want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("name", golden_util.names())
def test_ggml_restatement_within_tolerance_of_fixture(name):
    c, want = golden_util.load(name)
    got = cases.oracle_ggml(c)
    assert float(np.abs(got - want).max()) <= ATOL
    den = np.linalg.norm(want)
    assert np.linalg.norm(got - want) <= RTOL * den + 1e-12
