"""The residual add + RMSNorm fused into the projection that reads it
(cuca_hip_add_rmsnorm_qmm, _qmm_glu, _qmm_rope_store_kv), through the C ABI.

Bar: bit-exact against the two calls it replaces -- cuca_hip_add_rmsnorm into
x' and h, then cuca_hip_qmm / _qmm_glu / _qmm_rope_store_kv on h -- for x', h
and every matmul output.  At one activation row the matmul's workgroups
compute the norm themselves, replaying the norm kernel's summation order for
its thread shape, so the sizes cover every shape class of that kernel: fewer
than 64 threads a row (hidden 32, 96), one wave (256), several waves (544,
2048), 1024 threads (4096) and 1024 threads of 2 and 4 chunks (4128, 8192,
14336 f32), in f32 and f16 (8 values a chunk), with and without the branch,
the norm weights, the residual scale and x_out.  The matmul bits themselves
are pinned against the oracle: the fused output equals the oracle's qmm of
the fused h.  Also: two rows and a row past the one-row kernel's LDS (16384
f16: the two-launch path), the launch count at one row, and the overlap
error.
"""
import numpy as np
import pytest

from cuca_amd import hip
from helpers import assert_bits_equal
from oracle import oracle as O
from test_gpu_qmm import NP, QT, weight

pytestmark = pytest.mark.gpu


def inputs(ctx, rng, m, k, dtype, branch=True, norm_w=True):
    x = (rng.standard_normal((m, k)) * 2.0).astype(NP[dtype])
    b = (rng.standard_normal((m, k)) * 2.0).astype(NP[dtype]) if branch else None
    w = (1 + 0.05 * rng.standard_normal(k)).astype(np.float32) if norm_w else None
    dx = ctx.array(x)
    db = None if b is None else ctx.array(b)
    dw = None if w is None else ctx.array(w)
    return x, dx, db, dw


def ref_norm(ctx, dx, db, dw, eps, rs, m, k, dtype):
    """cuca_hip_add_rmsnorm into fresh x' and h."""
    xo = ctx.empty((m, k), NP[dtype])
    h = ctx.empty((m, k), NP[dtype])
    ctx.add_rmsnorm(dx.ptr, None if db is None else db.ptr, None if dw is None else dw.ptr, None, eps, eps, rs,
                    m, k, xo.ptr, h.ptr, hip.dtype_code(NP[dtype]))
    return xo, h


def ptr(a):
    return None if a is None else a.ptr


def launches(ctx, call):
    """The kernels one call launches."""
    ctx.sync()
    ctx.profile_start(8)
    call()
    recs = ctx.profile_stop()
    ctx.check_device()
    return [k for k, _ in recs]


CASES = [  # (k, dtype): every thread-shape class of the norm kernel
    (32, "f32"), (96, "f32"), (256, "f32"), (544, "f32"), (2048, "f32"), (4096, "f32"), (4128, "f32"),
    (8192, "f32"), (14336, "f32"), (96, "f16"), (4096, "f16"), (8192, "f16"), (16384, "f16")]


@pytest.mark.parametrize("k,dtype", CASES)
@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_plain_is_norm_then_qmm(ctx, k, dtype, qtype):
    rng = np.random.default_rng(k * 3 + len(dtype) + len(qtype))
    m, n, eps = 1, 37, 1e-5
    raw, w = weight(ctx, rng, qtype, n, k)
    x, dx, db, dw = inputs(ctx, rng, m, k, dtype)
    wx, wh = ref_norm(ctx, dx, db, dw, eps, 1.0, m, k, dtype)
    want = ctx.empty((m, n), NP[dtype])
    ctx.qmm(w.packed.ptr, QT[qtype], n, k, wh.ptr, k, m, n, want.ptr, n, hip.dtype_code(NP[dtype]))
    xo, h, out = ctx.empty((m, k), NP[dtype]), ctx.empty((m, k), NP[dtype]), ctx.empty((m, n), NP[dtype])
    names = launches(ctx, lambda: ctx.add_rmsnorm_qmm(dx.ptr, db.ptr, dw.ptr, eps, 1.0, xo.ptr, h.ptr, w.packed.ptr,
                                                      QT[qtype], n, k, m, n, out.ptr, n,
                                                      hip.dtype_code(NP[dtype])))
    if k < 16384:
        assert len(names) == 1 and "_rn" in names[0], names
    else:  # the expanded row outgrows the one-row kernel's LDS: the norm, then the chunked matmul
        assert len(names) == 2 and names[0].startswith("cuca_norm"), names
    assert_bits_equal(xo.numpy(), wx.numpy(), f"x' {k} {dtype}")
    assert_bits_equal(h.numpy(), wh.numpy(), f"h {k} {dtype}")
    got = out.numpy()
    assert_bits_equal(got, want.numpy(), f"out {k} {dtype} {qtype}")
    if dtype == "f32":  # the matmul's bits: the oracle's qmm of h
        assert_bits_equal(got, O.qmm(raw, QT[qtype], n, k, h.numpy(), rows=n, threads=8), "oracle qmm of h")


@pytest.mark.parametrize("branch,norm_w,rs,x_out", [(False, True, 1.0, False), (True, False, 1.0, True),
                                                    (True, True, 0.5, True), (True, True, 1.0, False)])
@pytest.mark.parametrize("k,dtype", [(4096, "f32"), (544, "f16"), (8192, "f32")])
def test_glu_options(ctx, branch, norm_w, rs, x_out, k, dtype):
    rng = np.random.default_rng(k + 7 * branch + 3 * norm_w + int(4 * rs) + x_out)
    m, ff, eps, qtype = 1, 50, 1e-6, "q4_0"
    _, gw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    _, uw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    x, dx, db, dw = inputs(ctx, rng, m, k, dtype, branch, norm_w)
    wx, wh = ref_norm(ctx, dx, db, dw, eps, rs, m, k, dtype)
    dt = hip.dtype_code(NP[dtype])
    want = ctx.empty((m, ff), NP[dtype])
    ctx.qmm_glu(gw.packed.ptr, uw.packed.ptr, QT[qtype], ff, k, wh.ptr, k, m, hip.ACT_SILU, 0.0, want.ptr, ff, dt)
    xo = ctx.empty((m, k), NP[dtype]) if x_out else None
    h, out = ctx.empty((m, k), NP[dtype]), ctx.empty((m, ff), NP[dtype])
    names = launches(ctx, lambda: ctx.add_rmsnorm_qmm_glu(dx.ptr, ptr(db), ptr(dw), eps, rs, ptr(xo), h.ptr,
                                                          gw.packed.ptr, uw.packed.ptr, QT[qtype], ff, k, m,
                                                          hip.ACT_SILU, 0.0, out.ptr, ff, dt))
    assert len(names) == 1 and names[0].startswith("cuca_qmd_glu") and "_rn" in names[0], names
    if x_out:
        assert_bits_equal(xo.numpy(), wx.numpy(), "x'")
    assert_bits_equal(h.numpy(), wh.numpy(), "h")
    assert_bits_equal(out.numpy(), want.numpy(), "glu out")


@pytest.mark.parametrize("act,clamp", [(hip.ACT_GELU_TANH, 0.0), (hip.ACT_SILU, 1.5)])
@pytest.mark.parametrize("m", [1, 2])
def test_glu_act_clamp_and_two_rows(ctx, act, clamp, m):
    """GeGLU and the clamp; two rows take the norm launch and the matmul."""
    rng = np.random.default_rng(act * 10 + m)
    k, ff, eps, qtype, dtype = 4096, 70, 1e-5, "q8_0", "f32"
    _, gw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    _, uw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    x, dx, db, dw = inputs(ctx, rng, m, k, dtype)
    wx, wh = ref_norm(ctx, dx, db, dw, eps, 1.0, m, k, dtype)
    dt = hip.dtype_code(NP[dtype])
    want = ctx.empty((m, ff), NP[dtype])
    ctx.qmm_glu(gw.packed.ptr, uw.packed.ptr, QT[qtype], ff, k, wh.ptr, k, m, act, clamp, want.ptr, ff, dt)
    xo, h, out = ctx.empty((m, k), NP[dtype]), ctx.empty((m, k), NP[dtype]), ctx.empty((m, ff), NP[dtype])
    names = launches(ctx, lambda: ctx.add_rmsnorm_qmm_glu(dx.ptr, db.ptr, dw.ptr, eps, 1.0, xo.ptr, h.ptr,
                                                          gw.packed.ptr, uw.packed.ptr, QT[qtype], ff, k, m, act,
                                                          clamp, out.ptr, ff, dt))
    assert len(names) == m, names  # one row: one launch; two: the norm, then the matmul
    assert_bits_equal(xo.numpy(), wx.numpy(), "x'")
    assert_bits_equal(h.numpy(), wh.numpy(), "h")
    assert_bits_equal(out.numpy(), want.numpy(), "glu out")


@pytest.mark.parametrize("k,dtype,qtype", [(4096, "f32", "q4_0"), (4096, "f16", "q8_0"), (8192, "f32", "q4_0"),
                                           (2048, "f32", "q8_0")])
def test_glu_eight_wave_workgroups(ctx, k, dtype, qtype):
    """A GLU of at least 32 rows per compute unit runs as 8-wave workgroups
    (one activation item a thread to 4096 values): the same bits."""
    rng = np.random.default_rng(k + len(dtype) + len(qtype))
    m, ff, eps = 1, 8200, 1e-5
    _, gw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    _, uw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    x, dx, db, dw = inputs(ctx, rng, m, k, dtype)
    wx, wh = ref_norm(ctx, dx, db, dw, eps, 1.0, m, k, dtype)
    dt = hip.dtype_code(NP[dtype])
    want = ctx.empty((m, ff), NP[dtype])
    names = launches(ctx, lambda: ctx.qmm_glu(gw.packed.ptr, uw.packed.ptr, QT[qtype], ff, k, wh.ptr, k, m,
                                              hip.ACT_SILU, 0.0, want.ptr, ff, dt))
    assert names == [f"cuca_qmd_glu_{dtype}_{qtype}_silu_n{2 if k <= 4096 else 8}w8"], names
    xo, h, out = ctx.empty((m, k), NP[dtype]), ctx.empty((m, k), NP[dtype]), ctx.empty((m, ff), NP[dtype])
    names = launches(ctx, lambda: ctx.add_rmsnorm_qmm_glu(dx.ptr, db.ptr, dw.ptr, eps, 1.0, xo.ptr, h.ptr,
                                                          gw.packed.ptr, uw.packed.ptr, QT[qtype], ff, k, m,
                                                          hip.ACT_SILU, 0.0, out.ptr, ff, dt))
    assert len(names) == 1 and names[0].endswith("w8_rn"), names
    assert_bits_equal(xo.numpy(), wx.numpy(), "x'")
    assert_bits_equal(h.numpy(), wh.numpy(), "h")
    assert_bits_equal(out.numpy(), want.numpy(), "glu out")


@pytest.mark.parametrize("qtype,dtype,k", [("q8_0", "f32", 4096), ("q4_0", "f16", 2048), ("q4_0", "f32", 8192)])
def test_tall_plain_the_final_norm_and_head(ctx, qtype, dtype, k):
    """The final norm in front of the LM head: a plain matmul of at least 32
    rows per compute unit runs as 8-wave workgroups with the prologue."""
    rng = np.random.default_rng(k + len(qtype))
    m, n, eps = 1, 9000, 1e-5
    raw, w = weight(ctx, rng, qtype, n, k)
    x, dx, db, dw = inputs(ctx, rng, m, k, dtype)
    wx, wh = ref_norm(ctx, dx, db, dw, eps, 1.0, m, k, dtype)
    dt = hip.dtype_code(NP[dtype])
    want = ctx.empty((m, n), NP[dtype])
    ctx.qmm(w.packed.ptr, QT[qtype], n, k, wh.ptr, k, m, n, want.ptr, n, dt)
    h, out = ctx.empty((m, k), NP[dtype]), ctx.empty((m, n), NP[dtype])
    names = launches(ctx, lambda: ctx.add_rmsnorm_qmm(dx.ptr, db.ptr, dw.ptr, eps, 1.0, None, h.ptr, w.packed.ptr,
                                                      QT[qtype], n, k, m, n, out.ptr, n, dt))
    assert names == [f"cuca_qmd_{dtype}_{qtype}_n{2 if k <= 4096 else 8}w8_rn"], names
    assert_bits_equal(h.numpy(), wh.numpy(), "h")
    got = out.numpy()
    assert_bits_equal(got, want.numpy(), "head out")
    if dtype == "f32":
        assert_bits_equal(got, O.qmm(raw, QT[qtype], n, k, h.numpy(), rows=n, threads=8), "oracle qmm of h")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d,k,m", [(32, 8, 128, 4096, 1), (4, 2, 64, 512, 1), (4, 2, 64, 512, 3),
                                         (6, 2, 64, 8192, 1)])
def test_qkv_rope_store(ctx, qtype, dtype, nq, nk, d, k, m):
    """At one row the 8-wave kernels (rows to 4096 values, and beyond)."""
    rng = np.random.default_rng(nq + nk + d + k + m + len(qtype))
    n, eps = (nq + 2 * nk) * d, 1e-5
    _, w = weight(ctx, rng, qtype, n, k)
    x, dx, db, dw = inputs(ctx, rng, m, k, dtype)
    dt = hip.dtype_code(NP[dtype])
    n_blocks = 8 + m
    cos, sin = hip.rope_tables(hip.ROPE_NORM, d, 5e5, 8192)
    dcos, dsin = ctx.array(cos), ctx.array(sin)
    dpos = ctx.array(rng.integers(0, 8192, m).astype(np.int32))
    dslots = ctx.array(rng.permutation(n_blocks * 16)[:m].astype(np.int32))
    init = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])

    def run(fused):
        pk, pv = ctx.array(init), ctx.array(init)
        q = ctx.empty((m, nq * d), NP[dtype])
        xo, h = ctx.empty((m, k), NP[dtype]), ctx.empty((m, k), NP[dtype])
        if fused:
            names = launches(ctx, lambda: ctx.add_rmsnorm_qmm_rope_store_kv(
                dx.ptr, db.ptr, dw.ptr, eps, 1.0, xo.ptr, h.ptr, w.packed.ptr, QT[qtype], k, m, nq, nk, d, d,
                hip.ROPE_NORM, dcos.ptr, dsin.ptr, 8192, dpos.ptr, q.ptr, nq * d, pk.ptr, pv.ptr, n_blocks,
                dslots.ptr, dt))
            assert len(names) == (1 if m == 1 else 2), names
            if m == 1:
                assert names[0].endswith("w8_rn"), names
        else:
            ctx.add_rmsnorm(dx.ptr, db.ptr, dw.ptr, None, eps, eps, 1.0, m, k, xo.ptr, h.ptr, dt)
            ctx.qmm_rope_store_kv(w.packed.ptr, QT[qtype], k, h.ptr, k, m, nq, nk, d, d, hip.ROPE_NORM, dcos.ptr,
                                  dsin.ptr, 8192, dpos.ptr, q.ptr, nq * d, pk.ptr, pv.ptr, n_blocks, dslots.ptr, dt)
        ctx.check_device()
        return [a.numpy() for a in (xo, h, q, pk, pv)]

    for name, got, want in zip(("x'", "h", "q", "pool k", "pool v"), run(True), run(False)):
        assert_bits_equal(got, want, f"{name} {qtype} {dtype} m={m}")


def test_outputs_must_not_overlap_inputs(ctx):
    rng = np.random.default_rng(5)
    k, n, dtype, qtype = 512, 16, "f32", "q4_0"
    _, w = weight(ctx, rng, qtype, n, k)
    x, dx, db, dw = inputs(ctx, rng, 1, k, dtype)
    h, out = ctx.empty((1, k), np.float32), ctx.empty((1, n), np.float32)
    dt = hip.dtype_code(np.float32)
    for xo, hh in ((dx, h), (db, h), (None, dx), (h, h)):
        with pytest.raises(hip.CucaError, match="overlap"):
            ctx.add_rmsnorm_qmm(dx.ptr, db.ptr, dw.ptr, 1e-5, 1.0, ptr(xo), hh.ptr, w.packed.ptr, QT[qtype], n, k,
                                1, n, out.ptr, n, dt)
    # no output written, and a good call still works afterwards
    ctx.add_rmsnorm_qmm(dx.ptr, db.ptr, dw.ptr, 1e-5, 1.0, None, h.ptr, w.packed.ptr, QT[qtype], n, k, 1, n,
                        out.ptr, n, dt)
    ctx.check_device()
