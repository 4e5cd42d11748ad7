"""The matrix-core quantized matmul (cuca_hip_qgemm, cuca_hip_qgemm_glu)
against the exact product, through the C ABI.

The arithmetic is the reference GPU engine's class for its dense paths
(float products of dequantised weights and unquantised activations,
moe_kernel.rs:1414-1600), not the CPU engine's bits: each weight is
f16(d * q), each activation f16(x), the products summed in f32.  Bar, per
output, against the f64 product of the oracle's dequantised weights
(dequant_row, the GGUF definition pinned by the golden rows) and the
activations:
    |got - want| <= (2^-10 + k 2^-24) * sum_i |w_i x_i|    (+ 2^-11 |want| for f16 output)
and for the GLU the same bounds carried through act(g) * u (|act'| <= 1.2).
A wrong pairing of weight and activation slots misses this by orders of
magnitude.  Covers Q4_0 / Q8_0, f32 / f16, 1 to 300 rows (tiles of 32, 64
and 128), rows that are not whole blocks of a packing group (k 96, 768),
weight-row prefixes and the host's argument errors.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

QT = {"q4_0": hip.GGML_Q4_0, "q8_0": hip.GGML_Q8_0}
NP = {"f32": np.float32, "f16": np.float16}


def dense(raw, qtype, n, k):
    rb = W.row_bytes(qtype, k)
    return np.stack([O.dequant_row(QT[qtype], raw[i * rb:(i + 1) * rb], 1.0, k) for i in range(n)]).astype(np.float64)


def bound(x, w, k):
    return (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(x) @ np.abs(w).T)


def setup(ctx, qtype, n, k, m, dtype, seed):
    rng = np.random.default_rng(seed)
    raw = W.quant_table(rng, n, k, qtype, (0.004, 0.03))
    wt = ops.QmmWeight.from_raw(ctx, QT[qtype], raw, n, k)
    x = (rng.standard_normal((m, k)) * 2).astype(NP[dtype])
    return raw, wt, x


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("n,k,m", [(130, 512, 1), (40, 4096, 5), (257, 768, 32), (64, 96, 33),
                                   (300, 2048, 64), (129, 1024, 100), (200, 512, 128), (96, 256, 300)])
def test_qgemm_within_the_bound(ctx, qtype, dtype, n, k, m):
    raw, wt, x = setup(ctx, qtype, n, k, m, dtype, n * 7 + k + m)
    dx = ctx.array(x)
    out = ctx.empty((m, n), NP[dtype])
    wsb = hip.qgemm_workspace(QT[qtype], n, k, m)
    ws = ctx.empty((wsb,), np.uint8)
    ctx.qgemm(wt.packed.ptr, QT[qtype], n, k, dx.ptr, k, m, n, ws.ptr, wsb, out.ptr, n, hip.dtype_code(NP[dtype]))
    got = out.numpy().astype(np.float64)
    w = dense(raw, qtype, n, k)
    xf = x.astype(np.float64)
    want = xf @ w.T
    tol = bound(xf, w, k) + (2.0 ** -11 * np.abs(want) if dtype == "f16" else 0.0) + 1e-30
    err = np.abs(got - want)
    assert np.all(err <= tol), (float(np.max(err / tol)), np.unravel_index(np.argmax(err / tol), err.shape))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("act,clamp", [(hip.ACT_SILU, 0.0), (hip.ACT_GELU_TANH, 0.0), (hip.ACT_SILU, 3.0)])
@pytest.mark.parametrize("m", [7, 64, 200])
def test_qgemm_glu_within_the_bound(ctx, qtype, act, clamp, m):
    n, k = 160, 1536
    rng = np.random.default_rng(m + act * 10 + int(clamp))
    graw = W.quant_table(rng, n, k, qtype, (0.004, 0.03))
    uraw = W.quant_table(rng, n, k, qtype, (0.004, 0.03))
    gw = ops.QmmWeight.from_raw(ctx, QT[qtype], graw, n, k)
    uw = ops.QmmWeight.from_raw(ctx, QT[qtype], uraw, n, k)
    x = (rng.standard_normal((m, k)) * 0.5).astype(np.float32)
    dx = ctx.array(x)
    out = ctx.empty((m, n), np.float32)
    wsb = hip.qgemm_workspace(QT[qtype], n, k, m, glu=True)
    ws = ctx.empty((wsb,), np.uint8)
    ctx.qgemm_glu(gw.packed.ptr, uw.packed.ptr, QT[qtype], n, k, dx.ptr, k, m, act, clamp, ws.ptr, wsb, out.ptr, n,
                  hip.F32)
    xf = x.astype(np.float64)
    wg, wu = dense(graw, qtype, n, k), dense(uraw, qtype, n, k)
    g, u = xf @ wg.T, xf @ wu.T
    bg, bu = bound(xf, wg, k), bound(xf, wu, k)
    if clamp > 0:
        g, u = np.minimum(g, clamp), np.clip(u, -clamp, clamp)
    if act == hip.ACT_SILU:
        a = g / (1.0 + np.exp(-g))
    else:
        a = 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))
    want = a * u
    tol = 1.2 * bg * (np.abs(u) + bu) + np.abs(a) * bu + 1e-5 * np.abs(want) + 1e-30
    err = np.abs(out.numpy().astype(np.float64) - want)
    assert np.all(err <= tol), float(np.max(err / tol))


def test_qgemm_weight_row_prefix_split_and_errors(ctx):
    """A prefix of the weight rows; the same product with k split (a full
    workspace) and unsplit (one that holds only the activations), both
    within the bound; a repeated call gives the same bits; the host's
    errors."""
    raw, wt, x = setup(ctx, "q8_0", 300, 4096, 40, "f32", 5)
    dx = ctx.array(x)
    out = ctx.empty((40, 100), np.float32)
    wsb = hip.qgemm_workspace(hip.GGML_Q8_0, 300, 4096, 40)
    ws = ctx.empty((wsb,), np.uint8)
    ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 40, 100, ws.ptr, wsb, out.ptr, 100, hip.F32)
    w = dense(raw, "q8_0", 300, 4096)[:100]
    want = x.astype(np.float64) @ w.T
    got = out.numpy()
    assert np.all(np.abs(got - want) <= bound(x.astype(np.float64), w, 4096) + 1e-30)
    small = (64 * 4096 * 2 + 255) // 256 * 256  # the activations, padded to a whole tile of 64 rows
    out2 = ctx.empty((40, 100), np.float32)
    ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 40, 100, ws.ptr, small, out2.ptr, 100, hip.F32)
    assert np.all(np.abs(out2.numpy() - want) <= bound(x.astype(np.float64), w, 4096) + 1e-30)
    out3 = ctx.empty((40, 100), np.float32)
    ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 40, 100, ws.ptr, wsb, out3.ptr, 100, hip.F32)
    assert np.array_equal(out3.numpy().view(np.uint32), got.view(np.uint32))
    with pytest.raises(hip.CucaError, match="weight rows"):
        ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 40, 301, ws.ptr, wsb, out.ptr, 400, hip.F32)
    with pytest.raises(hip.CucaError, match="output row stride"):
        ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 40, 100, ws.ptr, wsb, out.ptr, 99, hip.F32)
    with pytest.raises(hip.CucaError, match="workspace"):
        ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 40, 100, ws.ptr, small - 256, out.ptr, 100,
                  hip.F32)
    ctx.qgemm(wt.packed.ptr, hip.GGML_Q8_0, 300, 4096, dx.ptr, 4096, 0, 100, ws.ptr, wsb, out.ptr, 100, hip.F32)
