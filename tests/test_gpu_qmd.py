"""The decode matmul of one activation row (qmd.hip) against the oracle, through the C ABI.

cuca_hip_qmm, _qmm_glu and _qmm_rope_store_kv take this kernel for m = 1
whenever the row is at most 16384 values long; its arithmetic is the one-pass
kernel's, so the bars are test_gpu_qmm's: bit-exact against the oracle's
restatement of the CPU engine (qmm.rs) for the plain product (f16 output: the
oracle's f32 rounded once), the GLU's activation within cuca_hip_glu's bar,
and the fused Q|K|V epilogue equal to qmm followed by rope_store_kv and to
the oracle's qmm + rope + store.

Covers both row-length classes of the kernel (to 4096 values and to 16384),
rows that are not a multiple of the packing group (partial last groups: 17
and 129 blocks), group counts that are not a multiple of the ring depth,
weight-row counts that are not a multiple of a wave's four rows or a
workgroup's sixteen, weight-row prefixes, awkward activations (zero blocks,
ties, subnormal and huge values), the GLU's clamp, Q4_0 and Q8_0, f32 and
f16 activations, and the first row length past the kernel (16416, the
chunked kernel).
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O
from test_gpu_qmm import NP, QT, awkward, glu_floor, qkv_fused_vs_unfused, want_out, weight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("n,k", [(1, 32), (3, 96), (17, 544), (64, 2048), (130, 4096), (70, 4128),
                                 (33, 8192), (21, 14336), (5, 16384), (9, 16416)])
def test_one_row_is_bit_exact(ctx, qtype, dtype, n, k):
    rng = np.random.default_rng(n * 7 + k)
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, 1, k, huge=1e30 if dtype == "f32" else 1e4).astype(NP[dtype])
    got = w.forward(ctx.array(x)).numpy()
    assert_bits_equal(got, want_out(raw, qtype, n, k, x, n, dtype), f"{qtype} {dtype} {n}x{k}")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("k", [512, 4128])
def test_weight_row_prefix(ctx, qtype, k):
    rng = np.random.default_rng(k + 5)
    n = 40
    raw, w = weight(ctx, rng, qtype, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    for rows in (1, 5, 18, 37):
        got = w.forward_rows(ctx.array(x), rows).numpy()
        assert got.shape[-1] >= rows
        assert_bits_equal(got[..., :rows], want_out(raw, qtype, n, k, x, rows, "f32")[..., :rows],
                          f"{qtype} rows={rows}")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("ff,k,clamp", [(1, 32, 0.0), (37, 544, 0.0), (200, 4096, 2.0), (50, 14336, 0.0),
                                         (8200, 4096, 0.0), (8200, 4160, 1.0)])
def test_one_row_glu(ctx, qtype, dtype, act, ff, k, clamp):
    """(8200 rows: the 8-wave workgroups, a partial last one.)"""
    rng = np.random.default_rng(ff + k + act)
    graw, gw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    uraw, uw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    x = awkward(rng, 1, k, 1.0, huge=100.0).astype(NP[dtype])
    got = ops.QmmWeight.glu(gw, uw, ctx.array(x), ops.Glu(act, clamp)).numpy()
    g = O.qmm(graw, QT[qtype], ff, k, x, threads=8)
    u = O.qmm(uraw, QT[qtype], ff, k, x, threads=8)
    want = O.glu(g, u, act, clamp=clamp)
    gc = np.minimum(g, clamp) if clamp > 0 else g
    uc = np.clip(u, -clamp, clamp) if clamp > 0 else u
    want = want.astype(np.float16) if dtype == "f16" else want
    assert_close(got, want, floor=glu_floor(gc, uc, act), what=f"glu {qtype} {dtype} {ff}x{k}")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("ff,k,clamp", [(37, 544, 0.0), (50, 14336, 0.0), (8200, 4096, 0.0), (8200, 4160, 1.0)])
def test_one_row_glu_f16_finite(ctx, qtype, act, ff, k, clamp):
    """f16 outputs that all stay within f16 range (smaller weight scales than
    test_one_row_glu, whose Q8_0 cases overflow for a third of the rows), so
    the one-row GLU and its 8-wave form are checked on finite values."""
    rng = np.random.default_rng(3 * ff + k + act)
    graw, gw = weight(ctx, rng, qtype, ff, k, (0.001, 0.004))
    uraw, uw = weight(ctx, rng, qtype, ff, k, (0.001, 0.004))
    x = awkward(rng, 1, k, 1.0, huge=1.0).astype(np.float16)
    got = ops.QmmWeight.glu(gw, uw, ctx.array(x), ops.Glu(act, clamp)).numpy()
    g = O.qmm(graw, QT[qtype], ff, k, x, threads=8)
    u = O.qmm(uraw, QT[qtype], ff, k, x, threads=8)
    want = O.glu(g, u, act, clamp=clamp).astype(np.float16)
    assert np.all(np.isfinite(want))
    gc = np.minimum(g, clamp) if clamp > 0 else g
    uc = np.clip(u, -clamp, clamp) if clamp > 0 else u
    assert_close(got, want, floor=glu_floor(gc, uc, act), what=f"glu {qtype} f16 finite {ff}x{k}")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d,k", [(32, 8, 128, 4096), (4, 2, 64, 4128), (6, 2, 16, 256)])
def test_one_row_qkv_rope_store(ctx, qtype, dtype, nq, nk, d, k):
    rng = np.random.default_rng(nq * nk + d + k)
    raw, x, pos, slots, cos, sin, got_q, fpool = qkv_fused_vs_unfused(ctx, rng, qtype, dtype, nq, nk, d, k, 1)
    if dtype == "f32":
        n = (nq + 2 * nk) * d
        y = O.qmm(raw, QT[qtype], n, k, x, rows=n, threads=8)
        wq = O.rope(y[:, :nq * d].reshape(1, nq, d), cos, sin, pos, O.ROPE_NORM)
        assert_bits_equal(got_q.reshape(1, nq, d), wq, "oracle q")
        wk = O.rope(y[:, nq * d:(nq + nk) * d].reshape(1, nk, d), cos, sin, pos, O.ROPE_NORM)
        b, r = slots[0] // 16, slots[0] % 16
        assert_bits_equal(fpool.k.numpy()[b, :, r], wk[0], "oracle pool k")
        wv = y[:, (nq + nk) * d:].reshape(1, nk, d)
        assert_bits_equal(fpool.v.numpy()[b, :, r], wv[0], "oracle pool v")


def test_one_row_qkv_partial_rotary_and_bad_slot(ctx):
    rng = np.random.default_rng(91)
    qkv_fused_vs_unfused(ctx, rng, "q4_0", "f32", 4, 2, 64, 512, 1, n_dims=32)
    qkv_fused_vs_unfused(ctx, rng, "q8_0", "f32", 4, 2, 32, 256, 1, bad_row=0)


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m,n,k", [(1, 40, 544), (1, 24, 4128), (3, 40, 544), (2, 256 * 16 * 4 * 2, 64)])
def test_nan_activations_quantise_to_zero(ctx, qtype, m, n, k):
    """Acts::new: a NaN is ignored by the block maximum and quantises to 0
    (Rust's saturating `as i8`), so the outputs stay finite and equal the
    oracle's.  One row (the decode matmul), three (the one-pass kernel), and
    two rows of a tall matrix (the decode GEMV)."""
    rng = np.random.default_rng(m * 31 + k)
    raw, w = weight(ctx, rng, qtype, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, 5] = np.nan
    x[:, 32 + 31] = np.nan
    x[0, 34] = -np.nan
    got = w.forward(ctx.array(x)).numpy()
    want = want_out(raw, qtype, n, k, x, n, "f32")
    assert np.all(np.isfinite(want))
    assert_bits_equal(got, want, f"{qtype} m={m} {n}x{k} NaN activations")
