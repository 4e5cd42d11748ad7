"""Gated activation on the GPU against the oracle.

Bars: 1e-5 relative (f32) / 2 f16 ulps, plus for GELU-tanh the floor
2^-22 |0.5 g u| (candle's 1 + tanh(z) cancels for z << 0; the GPU's
2 sigma(2z) form does not).  Covers configs A-E (SiLU and GeGLU-tanh, f32
and f16, acts ~N(0, 1) and ~N(0, 2)), the clamp, the fused [gate | up]
layout, the ragged MoE rows with Zipf(1.1) expert offsets read on the
device, the generic kernel and the full config C size on sampled rows.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.float16}


def floor(g, u, act):
    if act != hip.ACT_GELU_TANH:
        return None
    return 2.0 ** -22 * np.abs(0.5 * g.astype(np.float64) * u.astype(np.float64))


def check(got, g, u, act, clamp=0.0, what=""):
    want = O.glu(g, u, act, clamp=clamp)
    gc = np.minimum(g.astype(np.float32), clamp) if clamp > 0 else g
    uc = np.clip(u.astype(np.float32), -clamp, clamp) if clamp > 0 else u
    assert_close(got, want, floor=floor(gc, uc, act), what=what)


@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("rows,ff,std", [(128, 3072, 1.0), (32, 14336, 1.0), (1, 14336, 1.0),
                                         (8, 14336, 2.0), (67, 768, 1.0), (3, 64, 8.0)])
def test_glu_matches_oracle(ctx, act, dtype, rows, ff, std):
    rng = np.random.default_rng(rows * 7 + ff + act)
    g = (std * rng.standard_normal((rows, ff))).astype(NP[dtype])
    u = rng.standard_normal((rows, ff)).astype(NP[dtype])
    got = ops.Glu(act).apply(ctx.array(g), ctx.array(u)).numpy()
    check(got, g, u, act, what=f"act {act} {dtype} {rows}x{ff}")


@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
def test_clamp(ctx, act):
    rng = np.random.default_rng(3)
    g = (3 * rng.standard_normal((16, 512))).astype(np.float32)
    u = (3 * rng.standard_normal((16, 512))).astype(np.float32)
    dg, du = ctx.array(g), ctx.array(u)
    plain = ops.Glu(act).apply(dg, du).numpy()
    for c in (0.5, 2.0, 10.0):
        got = ops.Glu.clamped(act, c).apply(dg, du).numpy()
        check(got, g, u, act, clamp=c, what=f"clamp {c}")
    assert np.array_equal(ops.Glu.clamped(act, 0.0).apply(dg, du).numpy(), plain)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_fused_gate_up_layout(ctx, dtype):
    rng = np.random.default_rng(4)
    ff = 3072
    y = rng.standard_normal((19, 2 * ff)).astype(NP[dtype])
    got = ops.Glu(hip.ACT_SILU).apply_fused(ctx.array(y), ff).numpy()
    check(got, y[:, :ff], y[:, ff:], hip.ACT_SILU, what="fused")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_ragged_moe_rows(ctx, dtype):
    rng = np.random.default_rng(5)
    n_tok, n_exp, k, ff = 64, 128, 8, 768
    offsets, tokens = W.zipf_expert_rows(rng, n_tok, n_exp, k)
    rows = int(offsets[-1])
    assert rows == n_tok * k and np.all(np.diff(offsets) >= 0)
    max_rows = rows + 40   # the buffer is sized for more rows than this call routes
    g = rng.standard_normal((max_rows, ff)).astype(NP[dtype])
    u = rng.standard_normal((max_rows, ff)).astype(NP[dtype])
    out = ctx.array(np.full((max_rows, ff), 7.0, NP[dtype]))
    ops.Glu(hip.ACT_SILU).apply_ragged(ctx.array(g), ctx.array(u), ctx.array(offsets), n_exp,
                                       out=out)
    got = out.numpy()
    check(got[:rows], g[:rows], u[:rows], hip.ACT_SILU, what="ragged")
    assert np.all(got[rows:] == 7.0)   # rows past offsets[n_experts] are not touched


@pytest.mark.parametrize("dtype,ff", [("f32", 99), ("f16", 100), ("f32", 3)])
def test_generic_kernel(ctx, dtype, ff):
    rng = np.random.default_rng(ff)
    for act in (hip.ACT_SILU, hip.ACT_GELU_TANH):
        g = (2 * rng.standard_normal((5, ff))).astype(NP[dtype])
        u = rng.standard_normal((5, ff)).astype(NP[dtype])
        got = ops.Glu(act).apply(ctx.array(g), ctx.array(u)).numpy()
        check(got, g, u, act, what=f"generic {dtype} {ff}")


def test_full_size_config_c_sampled_rows(ctx):
    torch = pytest.importorskip("torch")
    n, ff = 16384, 14336
    gen = torch.Generator(device="cuda").manual_seed(2)
    y = torch.randn((n, 2 * ff), device="cuda", generator=gen).to(torch.float16)
    out = torch.empty((n, ff), device="cuda", dtype=torch.float16)
    torch.cuda.synchronize()
    ctx.glu(y.data_ptr(), 2 * ff, y.data_ptr() + 2 * ff, 2 * ff, n, ff, hip.ACT_SILU, 0.0,
            out.data_ptr(), ff, hip.F16)
    ctx.sync()
    sample = torch.from_numpy(np.unique(np.concatenate(
        [[0, n - 1], np.random.default_rng(2).integers(0, n, 30)]))).cuda()
    ys = y[sample].cpu().numpy()
    check(out[sample].cpu().numpy(), ys[:, :ff], ys[:, ff:], hip.ACT_SILU, what="C full size")


@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_tails_underflow_like_the_reference(ctx, act, dtype):
    """Gate values out to +-100 and beyond: for g < -87 the reference's
    g / (1 + exp(-g)) passes through the f32 denormals to -0, and for large
    positive g it is g itself (no overflow in the kernel's rescaling)."""
    g = np.concatenate([np.linspace(-100.0, 100.0, 4093), [-1e30, 1e30, 3e38]]).astype(np.float32)
    g = g.reshape(4, -1).astype(NP[dtype]) if dtype == "f32" else \
        np.clip(g, -6e4, 6e4).reshape(4, -1).astype(np.float16)
    u = np.full(g.shape, 0.75, NP[dtype])
    got = ops.Glu(act).apply(ctx.array(g), ctx.array(u)).numpy()
    check(got, g, u, act, what=f"tails act {act} {dtype}")
