"""The dense f16 path for many rows (cuca_hip_qweight_dequant,
cuca_hip_gemm_w16, cuca_hip_gemm_w16_glu) through the C ABI.

- The dequantised copy is bit-exact: w16 = f16(d * q), the oracle's
  dequant_row (the GGUF definition pinned by the golden rows) rounded once
  to nearest-even.
- The GEMM is the arithmetic class of cuca_hip_qgemm (f16 weights and
  activations, f32 accumulation, here in the library's order) and is held to
  the same bar against the f64 product of the oracle's dequantised weights:
      |got - want| <= (2^-10 + k 2^-24) sum_i |w_i x_i|   (+ 2^-11 |want| for f16 output)
  and for the GLU the same bounds carried through act(g) * u.
Covers Q4_0 / Q8_0, f32 / f16 activations, 1 to 2048 rows (ragged tails of
rows and columns), weight-row prefixes, a row stride wider than k, repeated
calls, and the host's checks.  The GEMM is the library's own kernel
(gemm16.hip, cuca_gemm16_*): calls of fewer than 128 tiles of 256 x 256
(GLU: 128 columns) split k (the plain f32 form over every weight row, one
output matrix a split) and add the splits in a reduce launch; the GLU form
runs as 8 waves a workgroup, the plain form as 4.  Every form is covered, a
test pins which kernels a call launches, and one pins the GLU form's bits to
the plain form's sums put through the library's GLU op.
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
    return np.stack([O.dequant_row(QT[qtype], raw[i * rb:(i + 1) * rb], 1.0, k) for i in range(n)])


def bound(x, w, k):
    return (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(x) @ np.abs(w).T)


def dequantised(ctx, qtype, raw, n, k):
    wt = ops.QmmWeight.from_raw(ctx, QT[qtype], raw, n, k)
    w16 = ctx.empty((n, k), np.float16)
    ctx.qweight_dequant(wt.packed.ptr, QT[qtype], n, k, w16.ptr)
    return w16


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("n,k", [(3, 32), (17, 544), (64, 4096), (5, 14336)])
def test_dequant_is_bit_exact(ctx, qtype, n, k):
    rng = np.random.default_rng(n + k)
    raw = W.quant_table(rng, n, k, qtype, (0.0005, 0.05))
    got = dequantised(ctx, qtype, raw, n, k).numpy()
    want = dense(raw, qtype, n, k).astype(np.float32).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("n,k,m", [(130, 512, 1), (257, 768, 33), (300, 2048, 64), (96, 4096, 200),
                                   (512, 1024, 512), (300, 512, 1100), (520, 256, 2048)])
def test_gemm_within_the_bound(ctx, qtype, dtype, n, k, m):
    rng = np.random.default_rng(n * 7 + k + m)
    raw = W.quant_table(rng, n, k, qtype, (0.004, 0.03))
    w16 = dequantised(ctx, qtype, raw, n, k)
    ldx = k + 32
    x = (rng.standard_normal((m, ldx)) * 2).astype(NP[dtype])
    out = ctx.empty((m, n), NP[dtype])
    wsb = hip.gemm_w16_workspace(n, k, m, False, hip.dtype_code(NP[dtype]))
    ws = ctx.empty((wsb,), np.uint8)
    dx = ctx.array(x)
    ctx.gemm_w16(w16.ptr, n, k, dx.ptr, ldx, m, n, ws.ptr, wsb, out.ptr, n, hip.dtype_code(NP[dtype]))
    first = out.numpy()
    got = first.astype(np.float64)
    w = dense(raw, qtype, n, k).astype(np.float64)
    xf = x[:, :k].astype(np.float64)
    want = xf @ w.T
    tol = bound(xf, w, k) + (2.0 ** -11 * np.abs(want) if dtype == "f16" else 0.0) + 1e-30
    err = np.abs(got - want)
    assert np.all(err <= tol), (float(np.max(err / tol)), np.unravel_index(np.argmax(err / tol), err.shape))
    # the same call again: the same bits
    ctx.gemm_w16(w16.ptr, n, k, dx.ptr, ldx, m, n, ws.ptr, wsb, out.ptr, n, hip.dtype_code(NP[dtype]))
    assert np.array_equal(out.numpy().view(np.uint8), first.view(np.uint8))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("act,clamp", [(hip.ACT_SILU, 0.0), (hip.ACT_GELU_TANH, 0.0), (hip.ACT_SILU, 3.0)])
@pytest.mark.parametrize("m,ff", [(7, 160), (256, 160), (9, 162), (1030, 200)])
def test_gemm_glu_within_the_bound(ctx, qtype, dtype, act, clamp, m, ff):
    k = 1536
    rng = np.random.default_rng(m + act * 10 + int(clamp))
    graw = W.quant_table(rng, ff, k, qtype, (0.004, 0.03))
    uraw = W.quant_table(rng, ff, k, qtype, (0.004, 0.03))
    w16 = ctx.empty((2 * ff, k), np.float16)   # gate rows, then up rows
    for i, raw in enumerate((graw, uraw)):
        wt = ops.QmmWeight.from_raw(ctx, QT[qtype], raw, ff, k)
        ctx.qweight_dequant(wt.packed.ptr, QT[qtype], ff, k, w16.ptr + i * ff * k * 2)
    x = (rng.standard_normal((m, k)) * 0.5).astype(NP[dtype])
    dx = ctx.array(x)
    out = ctx.empty((m, ff), NP[dtype])
    wsb = hip.gemm_w16_workspace(ff, k, m, True, hip.dtype_code(NP[dtype]))
    ws = ctx.empty((wsb,), np.uint8)
    ctx.gemm_w16_glu(w16.ptr, ff, k, dx.ptr, k, m, act, clamp, ws.ptr, wsb, out.ptr, ff, hip.dtype_code(NP[dtype]))
    xf = x.astype(np.float64)
    wg, wu = dense(graw, qtype, ff, k).astype(np.float64), dense(uraw, qtype, ff, k).astype(np.float64)
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
    if dtype == "f16":
        tol = tol + 2.0 ** -11 * np.abs(want)
    err = np.abs(out.numpy().astype(np.float64) - want)
    assert np.all(err <= tol), float(np.max(err / tol))


def test_row_prefix_and_host_checks(ctx):
    rng = np.random.default_rng(9)
    n, k, m = 300, 1024, 40
    raw = W.quant_table(rng, n, k, "q8_0", (0.004, 0.03))
    w16 = dequantised(ctx, "q8_0", raw, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    dx = ctx.array(x)
    wsb = hip.gemm_w16_workspace(n, k, m, False, hip.F32)
    ws = ctx.empty((wsb,), np.uint8)
    full, part = ctx.empty((m, n), np.float32), ctx.empty((m, 100), np.float32)
    ctx.gemm_w16(w16.ptr, n, k, dx.ptr, k, m, n, ws.ptr, wsb, full.ptr, n, hip.F32)
    ctx.gemm_w16(w16.ptr, n, k, dx.ptr, k, m, 100, ws.ptr, wsb, part.ptr, 100, hip.F32)
    w = dense(raw, "q8_0", n, k).astype(np.float64)
    want = x.astype(np.float64) @ w[:100].T
    tol = bound(x.astype(np.float64), w[:100], k) + 1e-30
    assert np.all(np.abs(part.numpy() - want) <= tol)
    with pytest.raises(hip.CucaError, match="workspace of"):
        ctx.gemm_w16(w16.ptr, n, k, dx.ptr, k, m, n, ws.ptr, wsb - 1, full.ptr, n, hip.F32)
    with pytest.raises(hip.CucaError, match="weight rows"):
        ctx.gemm_w16(w16.ptr, n, k, dx.ptr, k, m, n + 1, ws.ptr, wsb, full.ptr, n + 1, hip.F32)
    with pytest.raises(hip.CucaError, match="row stride"):
        ctx.gemm_w16(w16.ptr, n, k, dx.ptr, k - 32, m, n, ws.ptr, wsb, full.ptr, n, hip.F32)


@pytest.mark.parametrize("m,n,k,glu,kernels", [
    (512, 4096, 4096, False, ["cuca_gemm16_f32", "cuca_gemm16_reduce_f16"]),   # 32 tiles: k split 8 ways
    (1024, 8192, 512, False, ["cuca_gemm16_f16"]),                          # 128 tiles: one pass
    (512, 2048, 1024, True, ["cuca_gemm16_f32", "cuca_gemm16_reduce_glu_f16_silu"]),
    (2048, 2048, 256, True, ["cuca_gemm16_w8_glu_f16_silu"]),               # the GLU form: 8 waves
])
def test_the_library_kernels_run(ctx, m, n, k, glu, kernels):
    """The dense GEMM is this library's kernel (no library GEMM underneath):
    the launched kernels by name, and the result within the bound on a few
    sampled rows."""
    rng = np.random.default_rng(m + n + k)
    rows = 2 * n if glu else n
    w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    dw, dx = ctx.array(w), ctx.array(x)
    out = ctx.empty((m, n), np.float16)
    wsb = hip.gemm_w16_workspace(n, k, m, glu, hip.F16)
    ws = ctx.empty((max(wsb, 16),), np.uint8)
    ctx.sync()
    ctx.profile_start(4)
    if glu:
        ctx.gemm_w16_glu(dw.ptr, n, k, dx.ptr, k, m, hip.ACT_SILU, 0.0, ws.ptr, wsb, out.ptr, n, hip.F16)
    else:
        ctx.gemm_w16(dw.ptr, n, k, dx.ptr, k, m, n, ws.ptr, wsb, out.ptr, n, hip.F16)
    names = [kn for kn, _ in ctx.profile_stop()]
    assert names == kernels, names
    sel = np.array([0, m // 3, m - 1])
    xf, wf = x[sel].astype(np.float64), w.astype(np.float64)
    got = out.numpy()[sel].astype(np.float64)
    if glu:
        g, u = xf @ wf[:n].T, xf @ wf[n:].T
        bg, bu = bound(xf, wf[:n], k), bound(xf, wf[n:], k)
        a = g / (1.0 + np.exp(-g))
        want = a * u
        tol = 1.2 * bg * (np.abs(u) + bu) + np.abs(a) * bu + 1e-5 * np.abs(want)
    else:
        want = xf @ wf.T
        tol = bound(xf, wf, k)
    tol = tol + 2.0 ** -11 * np.abs(want) + 1e-30
    assert np.all(np.abs(got - want) <= tol), float(np.max(np.abs(got - want) / tol))


@pytest.mark.parametrize("m,n,k,glu", [(300, 257, 32, False), (5, 100, 64, False), (513, 300, 96, True),
                                       (260, 70, 160, True), (1, 9, 32, True)])
def test_short_k_and_ragged_tiles(ctx, m, n, k, glu):
    """k of one to five stages of 32 (fewer stages than the kernel keeps in
    flight), tiles cut by both m and n, odd output widths (element stores)."""
    rng = np.random.default_rng(m * 3 + n + k)
    rows = 2 * n if glu else n
    w = (rng.standard_normal((rows, k)) * 0.05).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    dw, dx = ctx.array(w), ctx.array(x)
    out = ctx.empty((m, n), np.float32)
    wsb = hip.gemm_w16_workspace(n, k, m, glu, hip.F32)
    ws = ctx.empty((max(wsb, 16),), np.uint8)
    xf32 = ctx.array(x.astype(np.float32))
    if glu:
        ctx.gemm_w16_glu(dw.ptr, n, k, xf32.ptr, k, m, hip.ACT_SILU, 0.0, ws.ptr, wsb, out.ptr, n, hip.F32)
    else:
        ctx.gemm_w16(dw.ptr, n, k, xf32.ptr, k, m, n, ws.ptr, wsb, out.ptr, n, hip.F32)
    xf, wf = x.astype(np.float64), w.astype(np.float64)
    got = out.numpy().astype(np.float64)
    if glu:
        g, u = xf @ wf[:n].T, xf @ wf[n:].T
        bg, bu = bound(xf, wf[:n], k), bound(xf, wf[n:], k)
        a = g / (1.0 + np.exp(-g))
        want = a * u
        tol = 1.2 * bg * (np.abs(u) + bu) + np.abs(a) * bu + 1e-5 * np.abs(want) + 1e-30
    else:
        want = xf @ wf.T
        tol = bound(xf, wf, k) + 1e-30
    assert np.all(np.abs(got - want) <= tol), float(np.max(np.abs(got - want) / tol))


def test_glu_form_bits_equal_plain_sums_through_the_glu_op(ctx):
    """The GLU form (8 waves) with f32 activations and output against the
    plain form (4 waves) over the same gate and up rows, whose f32 sums the
    library's GLU op (cuca_hip_glu) turns into act(g) * u: each sum adds the
    same products in the same order and act(g) * u is the same f32
    arithmetic, so the bits must agree, with and without the clamp."""
    rng = np.random.default_rng(6)
    m, ff, k = 2048, 2048, 512
    w = (rng.standard_normal((2 * ff, k)) * 0.05).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16).astype(np.float32)   # f16 values: rounded exactly
    dw, dx = ctx.array(w), ctx.array(x)
    wg = hip.gemm_w16_workspace(ff, k, m, True, hip.F32)
    wp = hip.gemm_w16_workspace(2 * ff, k, m, False, hip.F32)
    ws = ctx.empty((max(wg, wp),), np.uint8)
    for act, clamp in ((hip.ACT_SILU, 0.0), (hip.ACT_GELU_TANH, 0.0), (hip.ACT_SILU, 2.0)):
        glu_out = ctx.empty((m, ff), np.float32)
        ctx.profile_start(4)
        ctx.gemm_w16_glu(dw.ptr, ff, k, dx.ptr, k, m, act, clamp, ws.ptr, wg, glu_out.ptr, ff, hip.F32)
        assert [kn for kn, _ in ctx.profile_stop()] == [
            "cuca_cvt_f16_f32", "cuca_gemm16_w8_glu_f32_silu" if act == hip.ACT_SILU else "cuca_gemm16_w8_glu_f32_gelu"]
        sums = ctx.empty((m, 2 * ff), np.float32)
        ctx.profile_start(4)
        ctx.gemm_w16(dw.ptr, 2 * ff, k, dx.ptr, k, m, 2 * ff, ws.ptr, wp, sums.ptr, 2 * ff, hip.F32)
        assert [kn for kn, _ in ctx.profile_stop()] == ["cuca_cvt_f16_f32", "cuca_gemm16_f32"]
        ref = ctx.empty((m, ff), np.float32)
        ctx.glu(sums.ptr, 2 * ff, sums.ptr + ff * 4, 2 * ff, m, ff, act, clamp, ref.ptr, ff, hip.F32)
        assert np.array_equal(glu_out.numpy().view(np.uint32), ref.numpy().view(np.uint32)), (act, clamp)
