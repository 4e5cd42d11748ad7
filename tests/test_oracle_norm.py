"""Pins the oracle's residual add + RMSNorm (CPU only).

candle's rms_norm kernel is not vendored in the reference, so the bits of its
sequential f32 sum are not pinned; the oracle is pinned instead against:
- an f64 evaluation of the textbook formula, the reference's own test oracle
  `rms64` (cpu.rs:3906-3912), to 2e-6 relative;
- closed forms (constant rows, zero rows, eps), scale invariance;
- a planted mistake (mean over H - 1, eps outside the root) that the f64
  comparison must reject, so the check is known to have teeth.
"""
import numpy as np
import pytest

from oracle import oracle as O


def rms64(x, w, eps):
    """cpu.rs:3906-3912, vectorized: v / sqrt(mean(v^2) + eps) * w in f64."""
    x = x.astype(np.float64)
    m = np.sqrt((x * x).sum(-1, keepdims=True) / x.shape[-1] + eps)
    y = x / m
    return y if w is None else y * w.astype(np.float64)


def rel_err(got, want):
    want = np.asarray(want, np.float64)
    return np.max(np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), 1e-30))


@pytest.mark.parametrize("hidden,eps", [(1024, 1e-6), (4096, 1e-5), (3584, 1e-6), (2048, 1e-6),
                                        (128, 1e-6), (7, 1e-5)])
def test_rms_matches_f64(hidden, eps):
    rng = np.random.default_rng(hidden)
    x = rng.standard_normal((9, hidden)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    _, h = O.add_rmsnorm(x, None, w, eps, write_x=False)
    assert rel_err(h, rms64(x, w, eps)) < 2e-6


def test_residual_add_is_exact_and_norm_reads_the_sum():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    b = rng.standard_normal((5, 256)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    xo, h = O.add_rmsnorm(x, b, w, 1e-6)
    assert np.array_equal(xo, x + b)             # IEEE f32 add
    assert rel_err(h, rms64(x + b, w, 1e-6)) < 2e-6


def test_gemma_sandwich_and_residual_scale():
    rng = np.random.default_rng(2)
    x = (2 * rng.standard_normal((4, 3584))).astype(np.float32)
    b = (2 * rng.standard_normal((4, 3584))).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(3584)).astype(np.float32)
    wp = (1 + 0.02 * rng.standard_normal(3584)).astype(np.float32)
    xo, h = O.add_rmsnorm(x, b, w, 1e-6, w_post=wp, post_eps=1e-6, residual_scale=0.22)
    want_x = x.astype(np.float64) + 0.22 * rms64(b, wp, 1e-6)
    assert np.max(np.abs(xo - want_x)) < 4e-6 * np.max(np.abs(want_x))
    assert rel_err(h, rms64(xo, w, 1e-6)) < 2e-6


def test_closed_forms():
    c = np.float32(3.0)
    x = np.full((1, 64), c, np.float32)
    _, h = O.add_rmsnorm(x, None, None, 1e-5, write_x=False)
    want = np.float64(c) / np.sqrt(np.float64(c) ** 2 + 1e-5)
    assert abs(h[0, 0] - want) <= 2 * np.spacing(np.float32(want))
    z = np.zeros((2, 32), np.float32)
    _, hz = O.add_rmsnorm(z, None, np.ones(32, np.float32), 1e-6, write_x=False)
    assert np.all(hz == 0)   # eps keeps the root positive: no NaN


def test_scale_invariance():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    _, h1 = O.add_rmsnorm(x, None, None, 0.0, write_x=False)
    _, h2 = O.add_rmsnorm(x * np.float32(4.0), None, None, 0.0, write_x=False)
    assert np.array_equal(h1, h2)   # a power of two scales every rounding alike


def test_f16_rounds_once_and_reads_the_stored_sum():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 4096)).astype(np.float16)
    b = rng.standard_normal((6, 4096)).astype(np.float16)
    w = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    xo, h = O.add_rmsnorm(x, b, w, 1e-5)
    s32 = x.astype(np.float32) + b.astype(np.float32)
    assert np.array_equal(xo.view(np.uint16), s32.astype(np.float16).view(np.uint16))
    want = rms64(xo.astype(np.float32), w, 1e-5)
    got = h.astype(np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp)   # within one f16 ulp of the f64 value


def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    _, h = O.add_rmsnorm(x, None, None, 1e-6, write_x=False)
    x64 = x.astype(np.float64)
    wrong_n = x64 / np.sqrt((x64 ** 2).sum(-1, keepdims=True) / 1023 + 1e-6)
    assert rel_err(h, wrong_n) > 2e-6
    assert rel_err(h, rms64(x, None, 1e-6)) < 2e-6
    # eps only shows where the mean square is comparable to it
    xs = (x * np.float32(1e-3)).astype(np.float32)
    _, hs = O.add_rmsnorm(xs, None, None, 1e-6, write_x=False)
    xs64 = xs.astype(np.float64)
    wrong_eps = xs64 / (np.sqrt((xs64 ** 2).mean(-1, keepdims=True)) + 1e-6)
    assert rel_err(hs, wrong_eps) > 2e-6
    assert rel_err(hs, rms64(xs, None, 1e-6)) < 2e-6
