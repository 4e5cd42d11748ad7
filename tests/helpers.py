"""Tolerances and comparisons shared by the GPU parity tests.

The bars: the embedding gather and RoPE without a norm
are bit-exact; norm, activation and normed RoPE are within a maximum
relative error of 1e-5 in f32 and 2 ulp in f16 (against the f16 rounding of
the oracle), with these stated floors where the quantity is ill-conditioned:
- GELU-tanh: + 2^-22 * |0.5 g u|, the rounding of candle's 1 + tanh(z) term,
  which cancels for z << 0 (the GPU evaluates 2 sigma(2z), which does not);
- QK-normed RoPE: relative to the magnitude of the rotated pair
  sqrt(a'^2 + b'^2), the rotation's conditioning (a*c - b*s cancels);
- everything: + 1e-37 absolute, below the f32 normal range.
"""
import numpy as np


def _f64(a):
    return np.asarray(a).astype(np.float64)


def ulp16(v):
    with np.errstate(invalid="ignore", over="ignore"):
        return np.spacing(np.abs(_f64(v)).astype(np.float16)).astype(np.float64)


def pair_floor(want, kind_neox, n_dims):
    """1e-5 x the magnitude of each rotated pair of a QK-normed RoPE output,
    broadcast to its two values (a*c - b*s cancels; the rotation keeps the
    pair's magnitude)."""
    w = _f64(want)
    half = n_dims // 2
    a = np.arange(half) if kind_neox else 2 * np.arange(half)
    b = a + half if kind_neox else a + 1
    mag = np.zeros_like(w)
    m = np.hypot(w[..., a], w[..., b])
    mag[..., a], mag[..., b] = m, m
    return 1e-5 * mag


def assert_bits_equal(got, want, what=""):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    ib = np.uint16 if got.dtype == np.float16 else np.uint32
    g, w = got.view(ib), want.view(ib)
    bad = g != w
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} differ; first at {idx.tolist()}: "
                             f"got {got[tuple(idx[0])]!r} want {want[tuple(idx[0])]!r}")


# Raw (unfloored) errors of every assert_close of the session, for the
# summary conftest prints at the end of the run: (test, what, dtype, stats).
RAW = []
CURRENT_TEST = [""]


def nonfinite_mismatch(got, want):
    """Elements whose non-finite pattern differs from the oracle's: where
    `want` is NaN, `got` must be NaN; where `want` is +-inf, `got` must be
    the same-signed inf; where `want` is finite, `got` must be finite.  (A
    tolerance test alone passes all of these: |got - want| > tol is False
    whenever a NaN is involved, and an infinite `want` makes tol infinite.)"""
    g, w = _f64(got), _f64(want)
    return np.where(np.isnan(w), ~np.isnan(g),
                    np.where(np.isinf(w), g != w, ~np.isfinite(g)))


def error_stats(got, want, floor=None, rel=1e-5, ulps=2):
    """The error against the north star's plain bar, before any floor:
    f32 -> the maximum relative error |got - want| / |want|; f16 -> the
    maximum error in f16 ulps of want, over the elements where both are
    finite.  `floored` counts the elements within the bar only because of
    the floor (outside rel |want| or ulps ulp, inside the bar plus the
    floor); `nonfinite` counts the expected NaN/inf values (each checked
    for the same value), `nonfinite_bad` the elements whose non-finite
    pattern differs (nonfinite_mismatch)."""
    g, w = _f64(got), _f64(want)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        ok = np.isfinite(g) & np.isfinite(w)
        d = np.where(ok, np.abs(g - w), 0.0)
        f16 = np.asarray(got).dtype == np.float16
        if f16:
            u = ulp16(want)
            base = ulps * u
            err = np.where(ok & (u > 0), d / np.where(u > 0, u, 1.0), 0.0)
        else:
            base = rel * np.abs(w)
            err = np.where(ok, d / np.maximum(np.abs(w), 1e-30), 0.0)
        plain = base + 1e-37
        fl = 0.0 if floor is None else floor
        floored = int(np.count_nonzero(ok & (d > plain) & (d <= plain + fl)))
    return {"dtype": "f16" if f16 else "f32", "n": int(g.size),
            "max_ulp" if f16 else "max_rel": float(err.max()) if err.size else 0.0,
            "floored": floored, "nonfinite": int(np.count_nonzero(~np.isfinite(w))),
            "nonfinite_bad": int(np.count_nonzero(nonfinite_mismatch(g, w)))}


def assert_close(got, want, floor=None, rel=1e-5, ulps=2, what=""):
    """f32: |got - want| <= rel |want| + floor; f16: <= ulps * ulp16(want) +
    floor.  `want` is the oracle's output in the same dtype.  Returns the
    raw error statistics (error_stats) and records them for the session
    summary."""
    g, w = _f64(got), _f64(want)
    assert g.shape == w.shape, (g.shape, w.shape)
    with np.errstate(invalid="ignore", over="ignore"):
        if np.asarray(got).dtype == np.float16:
            tol = ulps * ulp16(want)
        else:
            tol = rel * np.abs(w)
        tol = tol + 1e-37
        if floor is not None:
            tol = tol + floor
        both = np.isfinite(g) & np.isfinite(w)
        bad = (both & (np.abs(g - w) > tol)) | nonfinite_mismatch(g, w)
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        nf = int(np.count_nonzero(nonfinite_mismatch(g, w)))
        with np.errstate(invalid="ignore", over="ignore"):
            fin = bad & np.isfinite(g) & np.isfinite(w)
            worst = np.max(np.abs(g - w)[fin] / np.maximum(tol[fin], 1e-300)) if fin.any() else 0.0
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance "
                             f"({nf} with a different NaN/inf pattern; worst finite {worst:.2f}x); "
                             f"first at {list(i)}: got {g[i]!r} want {w[i]!r}")
    st = error_stats(got, want, floor, rel, ulps)
    RAW.append((CURRENT_TEST[0], what, st))
    return st


def max_rel(got, want):
    g, w = _f64(got), _f64(want)
    return float(np.max(np.abs(g - w) / np.maximum(np.abs(w), 1e-30)))
