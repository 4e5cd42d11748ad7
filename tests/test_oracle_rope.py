"""Pins the oracle's RoPE tables and rotation (CPU only).

- The table tests of rope.rs:173-266 (definition, unit factors, linear
  scale, attention factor, YaRN blend), restated.
- The rotation case of cpu.rs:4336-4374 (heads 2, t 3, d 8, n_dims 6) against
  an independent formulation: complex multiplication in numpy.
- Invariants: pair norms are preserved, position 0 is the identity, NORM on a
  layout equals NEOX on the permuted layout (cpu.rs:4252-4276), and the
  inverse rotation restores the input.
- QK-norm + rotation against the f64 composition.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def test_plain_tables_match_the_definition():
    cos, sin = O.rope_tables(8, 10_000.0, 5)
    assert cos.shape == (5, 4)
    for pos in range(5):
        for i in range(4):
            theta = pos * 10_000.0 ** (-(2.0 * i) / 8.0)
            assert abs(cos[pos, i] - math.cos(theta)) < 1e-6
            assert abs(sin[pos, i] - math.sin(theta)) < 1e-6


def test_tables_are_f64_rounded_once():
    cos, sin = O.rope_tables(128, 5e5, 64)
    pos = np.arange(64, dtype=np.float64)[:, None]
    i0 = 2.0 * np.arange(64, dtype=np.float64)[None, :]
    theta = pos * np.power(5e5, -i0 / 128.0)
    # numpy's f64 pow/cos may differ from glibc in the last f64 bit, which
    # can move an f32 rounding by one ulp at most
    assert np.max(np.abs(cos - np.cos(theta).astype(np.float32)) / np.spacing(np.float32(1))) <= 1
    assert np.max(np.abs(sin - np.sin(theta).astype(np.float32)) / np.spacing(np.float32(1))) <= 1


def test_unit_factors_leave_pairs_unrotated():
    factors = np.concatenate([np.ones(64, np.float32), np.full(192, 1e30, np.float32)])
    cos, sin = O.rope_tables(512, 1e6, 4, factors=factors)
    assert np.all(cos[:, 64:] == 1.0)
    assert np.all(np.abs(sin[:, 64:]) < 1e-12)
    assert sin[1, 0] != 0.0


def test_linear_scale_and_attn_factor():
    base_c, _ = O.rope_tables(4, 100.0, 3)
    cos, _ = O.rope_tables(4, 100.0, 3, freq_scale=0.125)
    for pos in range(3):
        for i in range(2):
            theta = pos * 100.0 ** (-(2.0 * i) / 4.0) * 0.125
            assert abs(cos[pos, i] - math.cos(theta)) < 1e-6
    assert not np.array_equal(base_c, cos)
    c1, s1 = O.rope_tables(4, 100.0, 3)
    c2, s2 = O.rope_tables(4, 100.0, 3, attn_factor=1.5)
    assert np.max(np.abs(c1 * 1.5 - c2)) < 1e-6 and np.max(np.abs(s1 * 1.5 - s2)) < 1e-6


def test_yarn_blends_between_extrapolation_and_interpolation():
    factor = 4.0
    cos, _ = O.rope_tables(64, 10_000.0, 100, freq_scale=1 / factor, yarn=(1.0, 32.0, 1.0, 4096))
    mscale = 1.0 + 0.1 * math.log(factor)
    assert abs(cos[99, 0] - math.cos(99.0) * mscale) < 1e-5
    theta_last = 99 * 10_000.0 ** (-62.0 / 64.0) / factor
    assert abs(cos[99, 31] - math.cos(theta_last) * mscale) < 1e-5


def reference_case():
    heads, t, d, n_dims = 2, 3, 8, 6
    values = np.array([((i * 7 % 13) - 6.0) for i in range(heads * t * d)], np.float32)
    half = n_dims // 2
    cos = np.array([math.cos(i * 0.37) for i in range(t * half)], np.float32).reshape(t, half)
    sin = np.array([math.sin(i * 0.37) for i in range(t * half)], np.float32).reshape(t, half)
    # (1, heads, t, d) -> rows = t, heads: [t, heads, d]
    x = values.reshape(heads, t, d).transpose(1, 0, 2).copy()
    return x, cos, sin, n_dims


@pytest.mark.parametrize("kind", [O.ROPE_NORM, O.ROPE_NEOX])
def test_cpu_rs_4336_case_against_complex_multiplication(kind):
    x, cos, sin, n_dims = reference_case()
    got = O.rope(x, cos, sin, np.arange(3), kind, n_dims)
    half = n_dims // 2
    for p in range(3):
        for h in range(2):
            v = x[p, h].astype(np.float64)
            a_idx = np.arange(half) if kind == O.ROPE_NEOX else 2 * np.arange(half)
            b_idx = a_idx + half if kind == O.ROPE_NEOX else a_idx + 1
            z = (v[a_idx] + 1j * v[b_idx]) * (cos[p].astype(np.float64) + 1j * sin[p].astype(np.float64))
            want = v.copy()
            want[a_idx], want[b_idx] = z.real, z.imag
            assert np.max(np.abs(got[p, h] - want)) < 1e-5      # the reference's tolerance
            assert np.array_equal(got[p, h, n_dims:], x[p, h, n_dims:])


def test_invariants():
    rng = np.random.default_rng(7)
    rows, heads, d = 11, 3, 64
    x = rng.standard_normal((rows, heads, d)).astype(np.float32)
    cos, sin = O.rope_tables(d, 1e4, 40)
    pos = rng.integers(0, 40, rows).astype(np.int32)
    pos[0] = 0
    for kind in (O.ROPE_NORM, O.ROPE_NEOX):
        y = O.rope(x, cos, sin, pos, kind)
        assert np.array_equal(y[0], x[0])                       # position 0: identity
        a = np.arange(d // 2) if kind == O.ROPE_NEOX else 2 * np.arange(d // 2)
        b = a + d // 2 if kind == O.ROPE_NEOX else a + 1
        n0 = np.hypot(x[..., a].astype(np.float64), x[..., b].astype(np.float64))
        n1 = np.hypot(y[..., a].astype(np.float64), y[..., b].astype(np.float64))
        assert np.max(np.abs(n0 - n1) / np.maximum(n0, 1e-6)) < 1e-6
        back = O.rope(y, cos, -sin, pos, kind)                   # inverse rotation
        assert np.max(np.abs(back - x)) < 1e-5
    # NORM on a layout == NEOX on the permuted layout, bit for bit
    perm = np.concatenate([np.arange(0, d, 2), np.arange(1, d, 2)])
    y_norm = O.rope(x, cos, sin, pos, O.ROPE_NORM)
    y_neox = O.rope(x[..., perm], cos, sin, pos, O.ROPE_NEOX)
    assert np.array_equal(y_norm[..., perm], y_neox)
    # and the other pairing really is different
    assert not np.allclose(O.rope(x, cos, sin, pos, O.ROPE_NEOX), y_norm)


def test_qk_norm_then_rotation():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 4, 128)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    cos, sin = O.rope_tables(128, 1e6, 16)
    pos = np.arange(5, dtype=np.int32)
    got = O.rope(x, cos, sin, pos, O.ROPE_NEOX, norm_w=w, eps=1e-6)
    x64 = x.astype(np.float64)
    n = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    a, b = n[..., :64], n[..., 64:]
    c, s = cos[pos][:, None, :].astype(np.float64), sin[pos][:, None, :].astype(np.float64)
    want = np.concatenate([a * c - b * s, a * s + b * c], -1)
    assert np.max(np.abs(got - want)) < 1e-5


# ---------------------------------------------------------------------------
# the full-width QK-norm of the qk_norm_full archs (OLMo 2, OLMoE: cpu.rs:2838-2843
# for Q, 3042-3045 for K): rms over the whole projection row, then the rotation
# ---------------------------------------------------------------------------

def test_full_width_norm_is_the_row_norm_then_the_rotation():
    rng = np.random.default_rng(31)
    rows, heads, d = 7, 6, 32
    x = rng.standard_normal((rows, heads, d)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(heads * d)).astype(np.float32)
    cos, sin = O.rope_tables(d, 1e4, 16)
    pos = rng.integers(0, 16, rows).astype(np.int32)
    got = O.rope(x, cos, sin, pos, O.ROPE_NEOX, norm_w=w, eps=1e-6, full=True)
    _, h = O.add_rmsnorm(x.reshape(rows, heads * d), None, w, 1e-6, write_x=False)
    want = O.rope(h.reshape(rows, heads, d), cos, sin, pos, O.ROPE_NEOX)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # f64: normalise over the row, rotate the pairs
    x64 = x.astype(np.float64).reshape(rows, heads * d)
    n64 = (x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w).reshape(rows, heads, d)
    c, s = cos[pos].astype(np.float64)[:, None], sin[pos].astype(np.float64)[:, None]
    a, b = n64[..., : d // 2], n64[..., d // 2:]
    f64 = np.concatenate([a * c - b * s, a * s + b * c], -1)
    assert np.max(np.abs(got - f64)) < 2e-6 * np.max(np.abs(f64))


def test_full_width_norm_is_not_the_per_head_norm():
    """A planted mistake: the per-head norm with the same weights gives
    other values whenever the heads' scales differ."""
    rng = np.random.default_rng(32)
    rows, heads, d = 3, 4, 16
    x = (rng.standard_normal((rows, heads, d)) * np.array([1, 2, 4, 8])[None, :, None]).astype(np.float32)
    w = np.ones(heads * d, np.float32)
    cos, sin = O.rope_tables(d, 1e4, 4)
    pos = np.zeros(rows, np.int32)
    full = O.rope(x, cos, sin, pos, O.ROPE_NEOX, norm_w=w, full=True)
    per_head = O.rope(x, cos, sin, pos, O.ROPE_NEOX, norm_w=w[:d])
    assert np.max(np.abs(full - per_head)) > 0.1
    # position 0 rotates nothing: the full-width result is the row norm itself
    x64 = x.astype(np.float64).reshape(rows, -1)
    want = (x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6)).reshape(rows, heads, d)
    assert np.max(np.abs(full - want)) < 2e-6 * np.max(np.abs(want))
