"""Pins the oracle's rms_norm_rows (quant.rs:324-339), the scale-less norm
Hparams::norm_embeddings (params.rs:374-379) applies to the looked-up rows
of the embd_norm archs (CPU only).

- A pure-Python restatement on small rows -- the f64 squares folded in
  index order from 0, f64 division by the row length, the root and the
  reciprocal in f64, one rounding to f32, an f32 product -- gives the same
  bits.
- Closed forms: a row with one power-of-two value 2^k among 4096 zeros
  normalises to exactly 64 (mean 2^(2k-12), root 2^(k-6)); a constant row
  of 2^k normalises to exactly 1.
- A planted mistake, the squares summed in f32 (candle's rms_norm order),
  gives other bits on a row whose small squares vanish in an f32 sum; the
  f64 fold does not.
- The embedding with the norm is the gather, then the norm, then (f16) one
  rounding.
- The device's shortcut: it sums in another order and takes the f32 scale
  from an error bound when that decides it.  Restated here in numpy, it
  never decides a wrong value over thousands of random rows, and it declines
  the constructed rows the GPU test uses for the serial fallback.
"""
import math

import numpy as np
import pytest

from cuca_amd import workloads as W
from oracle import oracle as O


def norm_rows_py(rows, eps):
    out = np.empty_like(rows, dtype=np.float32)
    e = float(np.float32(eps))
    for r, row in enumerate(rows):
        s = 0.0
        for v in row:
            s += float(v) * float(v)
        inv = np.float32(1.0 / math.sqrt(s / len(row) + e))
        out[r] = row.astype(np.float32) * inv
    return out


def device_certified_inv(row, eps, order_seed=0):
    """The kernel's bound check (embed_norm_inv), in numpy f64: the squares
    summed in another order, then the f32 scale if the bound decides it,
    else None (the kernel then re-sums in index order)."""
    x = row.astype(np.float64)
    sq = x * x
    perm = np.random.default_rng(order_seed).permutation(sq.size)
    s = 0.0
    for v in sq[perm]:
        s += v
    n, e = float(row.size), float(np.float32(eps))
    b = s * (2.02 * n * 2.0 ** -53)
    lo = np.float32((1.0 / math.sqrt((s + b) / n + e)) * (1.0 - 2.0 ** -50))
    hi = np.float32((1.0 / math.sqrt((s - b) / n + e)) * (1.0 + 2.0 ** -50))
    return lo if lo == hi else None


@pytest.mark.parametrize("row_len,eps", [(32, 1e-6), (64, 1e-5), (96, 0.0), (256, 1e-6)])
def test_matches_the_sequential_f64_fold(row_len, eps):
    rng = np.random.default_rng(row_len)
    rows = (rng.standard_normal((5, row_len)) * rng.uniform(0.01, 50, (5, 1))).astype(np.float32)
    assert np.array_equal(O.rms_norm_rows(rows, eps).view(np.uint32),
                          norm_rows_py(rows, eps).view(np.uint32))


@pytest.mark.parametrize("k", [-9, -3, 0, 4])
def test_closed_forms(k):
    row = np.zeros((1, 4096), np.float32)
    row[0, 1234] = np.float32(2.0 ** k)
    out = O.rms_norm_rows(row, 0.0)
    assert out[0, 1234] == 64.0 and np.count_nonzero(out) == 1
    neg = O.rms_norm_rows(-row, 0.0)
    assert neg[0, 1234] == -64.0
    const = O.rms_norm_rows(np.full((1, 1024), 2.0 ** k, np.float32), 0.0)
    assert np.all(const == 1.0)


def test_planted_f32_sum_is_caught():
    row = np.full((1, 4096), 0.125, np.float32)
    row[0, 0] = 4096.0   # 4096^2 = 2^24: every 2^-6 square vanishes in an f32 sum
    got = O.rms_norm_rows(row, 1e-6)
    assert np.array_equal(got, norm_rows_py(row, 1e-6))
    s32 = np.float32(0.0)
    for v in row[0]:
        s32 = np.float32(s32 + np.float32(v * v))
    inv32 = np.float32(1.0 / math.sqrt(float(s32) / 4096 + float(np.float32(1e-6))))
    wrong = row * inv32
    assert not np.array_equal(got, wrong)


@pytest.mark.parametrize("ty,qname", [(O.Q4_0, "q4_0"), (O.Q8_0, "q8_0")])
@pytest.mark.parametrize("scale", [1.0, float(np.float32(math.sqrt(3584.0)))])
def test_embed_with_norm_is_gather_then_norm(ty, qname, scale):
    rng = np.random.default_rng(ty)
    hidden, vocab = 512, 64
    table = W.quant_table(rng, vocab, hidden, qname, (0.001, 0.05))
    ids = rng.integers(0, vocab, 9).astype(np.uint32)
    plain = O.embed(table, ty, vocab, hidden, ids, scale)
    want = O.rms_norm_rows(plain, 1e-6)
    got = O.embed(table, ty, vocab, hidden, ids, scale, norm_eps=1e-6)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = O.embed(table, ty, vocab, hidden, ids, scale, out_dtype=np.float16, norm_eps=1e-6)
    assert np.array_equal(got16.view(np.uint16), want.astype(np.float16).view(np.uint16))


def test_the_devices_bound_never_decides_a_wrong_scale():
    rng = np.random.default_rng(5)
    decided = 0
    for t in range(300):
        n = int(rng.choice([32, 256, 2048]))
        row = (rng.standard_normal(n) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        if t % 3 == 0:   # wide dynamic range
            row *= np.float32(2.0) ** rng.integers(-20, 20, n).astype(np.float32)
        eps = float(rng.choice([0.0, 1e-6, 1e-5]))
        inv = device_certified_inv(row, eps, order_seed=t)
        want = O.rms_norm_rows(row[None], eps)[0]
        if inv is not None:
            decided += 1
            assert np.array_equal(row * inv, want)
    assert decided >= 290


def fallback_case():
    """A Q8_0 row (d = 2^-7, exact squares and sums) and an eps whose scale
    sits so close to an f32 rounding midpoint that the device's bound cannot
    decide it: (table row bytes, eps)."""
    rng = np.random.default_rng(2024)
    hidden = 4096
    q = rng.integers(-127, 128, hidden).astype(np.int64)
    s = float((q * q).sum()) * 2.0 ** -14          # exact
    mean = s / hidden                              # exact (power of two)
    base = np.array([1e-5], np.float32).view(np.uint32)[0]
    eps32 = (base + np.arange(1 << 21, dtype=np.uint32)).view(np.float32)
    e = eps32.astype(np.float64)
    b = s * (2.02 * hidden * 2.0 ** -53)
    lo = ((1.0 / np.sqrt((s + b) / hidden + e)) * (1.0 - 2.0 ** -50)).astype(np.float32)
    hi = ((1.0 / np.sqrt((s - b) / hidden + e)) * (1.0 + 2.0 ** -50)).astype(np.float32)
    i = int(np.nonzero(lo != hi)[0][0])
    blocks = np.zeros((hidden // 32, 34), np.uint8)
    blocks[:, 0:2] = np.array([2.0 ** -7], np.float16).view(np.uint8)
    blocks[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(-1, 32)
    return blocks.reshape(-1), float(eps32[i])


def test_the_constructed_fallback_row_defeats_the_bound():
    row_bytes, eps = fallback_case()
    row = O.dequant_row(O.Q8_0, row_bytes, 1.0, 4096)
    assert device_certified_inv(row, eps) is None
    assert np.array_equal(O.rms_norm_rows(row[None], eps)[0], norm_rows_py(row[None], eps)[0])
