"""Pins the oracle's gated activation (CPU only).

candle's silu / gelu kernels are not vendored; the oracle is pinned against
f64 evaluations of the formulas the reference states (gpu.rs:5908-5913, the
f64 host `swiglu` of moe_kernel.rs:2340-2352 and `gelu64` of
cpu.rs:3913-3916), against the exact erf GELU that GELU-tanh approximates,
and against the clamp semantics of Glu::apply (cpu.rs:362-371).

Tolerance (relative, f32): 2e-6 for SiLU.  For GELU-tanh the candle form
0.5 g (1 + tanh z) cancels for z << 0, so the bound carries a floor of
2^-22 |0.5 g u| (two ulps of 1 on the 1 + tanh term).
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

K = math.sqrt(2.0 / math.pi)


def silu64(g):
    return g / (1.0 + np.exp(-g))


def gelu64(g):
    return 0.5 * g * (1.0 + np.tanh(K * (g + 0.044715 * g ** 3)))


def check(got, g, u, act):
    g = g.astype(np.float64)
    u = u.astype(np.float64)
    want = (silu64(g) if act == O.SILU else gelu64(g)) * u
    tol = 2e-6 * np.abs(want) + 1e-37
    if act == O.GELU_TANH:
        tol = tol + 2.0 ** -22 * np.abs(0.5 * g * u)
    bad = np.abs(got.astype(np.float64) - want) > tol
    assert not bad.any(), (g[bad][:4], got[bad][:4], want[bad][:4])


@pytest.mark.parametrize("act", [O.SILU, O.GELU_TANH])
@pytest.mark.parametrize("std", [1.0, 2.0, 8.0])
def test_matches_f64(act, std):
    rng = np.random.default_rng(int(std * 10) + act)
    g = (std * rng.standard_normal((16, 3072))).astype(np.float32)
    u = rng.standard_normal((16, 3072)).astype(np.float32)
    check(O.glu(g, u, act), g, u, act)


def test_gelu_tanh_approximates_erf_gelu():
    g = np.linspace(-6, 6, 4001).astype(np.float32)[None, :]
    u = np.ones_like(g)
    got = O.glu(g, u, O.GELU_TANH)[0].astype(np.float64)
    exact = np.array([0.5 * x * (1 + math.erf(x / math.sqrt(2))) for x in g[0].astype(np.float64)])
    assert np.max(np.abs(got - exact)) < 1e-3
    # dropping the cubic term or flipping the sign would not be within 1e-3
    no_cubic = 0.5 * g[0] * (1 + np.tanh(K * g[0]))
    assert np.max(np.abs(no_cubic - exact)) > 1e-2


def test_special_values():
    g = np.array([[0.0, -0.0, 30.0, -30.0, -100.0, 100.0]], np.float32)
    u = np.ones_like(g)
    s = O.glu(g, u, O.SILU)[0]
    assert s[0] == 0 and s[2] == 30.0 and s[5] == 100.0
    assert s[4] == 0 and np.signbit(s[4])     # -100 / (1 + inf) = -0
    gl = O.glu(g, u, O.GELU_TANH)[0]
    assert gl[0] == 0 and gl[2] == 30.0 and gl[3] == 0


def test_clamp_semantics():
    # gate clamped from above only, up to [-limit, limit]; 0 is no clamp
    g = np.array([[-5.0, 0.5, 3.0]], np.float32)
    u = np.array([[-9.0, 0.25, 9.0]], np.float32)
    c = O.glu(g, u, O.SILU, clamp=2.0)[0]
    sg = np.array([-5.0, 0.5, 2.0], np.float32)
    su = np.array([-2.0, 0.25, 2.0], np.float32)
    check(c[None, :], sg[None, :], su[None, :], O.SILU)
    assert np.array_equal(O.glu(g, u, O.SILU, clamp=0.0), O.glu(g, u, O.SILU))


def test_strided_fused_layout_and_f16():
    rng = np.random.default_rng(9)
    y = rng.standard_normal((7, 2 * 768)).astype(np.float32)
    out = O.glu(y[:, :768], y[:, 768:], O.SILU)
    assert np.array_equal(out, O.glu(np.ascontiguousarray(y[:, :768]),
                                     np.ascontiguousarray(y[:, 768:]), O.SILU))
    y16 = y.astype(np.float16)
    o16 = O.glu(y16[:, :768], y16[:, 768:], O.SILU)
    o32 = O.glu(y16[:, :768].astype(np.float32), y16[:, 768:].astype(np.float32), O.SILU)
    assert np.array_equal(o16.view(np.uint16), o32.astype(np.float16).view(np.uint16))
