"""The parity helpers themselves: planted mismatches must fail.

assert_close compares finite values to a tolerance and the rest by value:
an expected NaN needs a NaN, an expected +-inf the same-signed inf, and an
expected finite value a finite one.  Each case below plants one such
mismatch in otherwise identical arrays (f32 and f16)."""
import numpy as np
import pytest

from helpers import assert_close, error_stats, nonfinite_mismatch


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("got_v,want_v", [
    (np.nan, 1.0),      # a NaN where a finite value is expected
    (np.inf, 1.0),      # an overflow where a finite value is expected
    (1.0, np.inf),      # a finite value where the oracle overflows
    (5.0, -np.inf),
    (-np.inf, np.inf),  # the wrong sign of inf
    (np.inf, -np.inf),
    (3.0, np.nan),      # a finite value where the oracle's is NaN
    (np.inf, np.nan),
    (np.nan, np.inf),
])
def test_planted_nonfinite_mismatch_fails(dtype, got_v, want_v):
    want = np.linspace(-2, 2, 64).astype(dtype)
    got = want.copy()
    want[17], got[17] = want_v, got_v
    with pytest.raises(AssertionError, match="NaN/inf pattern"):
        assert_close(got, want, what="planted")
    st = error_stats(got, want)
    assert st["nonfinite_bad"] == 1


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_matching_nonfinite_values_pass(dtype):
    want = np.linspace(-2, 2, 64).astype(dtype)
    want[3], want[9], want[40] = np.inf, -np.inf, np.nan
    got = want.copy()
    got[40] = -np.nan  # any NaN payload or sign is a NaN
    st = assert_close(got, want, what="matching")
    assert st["nonfinite"] == 3 and st["nonfinite_bad"] == 0


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_planted_finite_error_fails(dtype):
    want = np.linspace(1, 2, 64).astype(dtype)
    got = want.copy()
    got[5] = dtype(float(want[5]) * (1 + 1e-2))  # 10 f16 ulps, 1e4 x the f32 bar
    with pytest.raises(AssertionError, match="outside tolerance"):
        assert_close(got, want, what="planted")


def test_floor_widens_only_finite_elements():
    want = np.array([1.0, np.inf, 2.0], np.float32)
    got = np.array([1.5, 1.0, 2.0], np.float32)
    floor = np.array([1.0, np.inf, 0.0])
    with pytest.raises(AssertionError, match="1 with a different NaN/inf"):
        assert_close(got, want, floor=floor, what="floor")
    assert nonfinite_mismatch(got, want).tolist() == [False, True, False]
