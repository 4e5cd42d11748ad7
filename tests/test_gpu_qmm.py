"""Quantized matmul (QmmWeight) on the GPU against the oracle, through the C ABI.

Bars:
- cuca_hip_qmm: bit-exact against the oracle's restatement of the reference
  CPU engine (qmm.rs), f32 output; f16 output is the oracle's f32 rounded
  once to nearest-even, bit-exact too;
- cuca_hip_qmm_glu: the gate and up products are those bits; the activation
  is held to cuca_hip_glu's bar (1e-5 relative in f32, 2 f16 ulps, plus for
  GELU-tanh the floor 2^-22 |0.5 g u|).
Covers Q4_0 and Q8_0, f32 and f16 activations, activation tiles of 1, 2 and
4 rows and ragged tails, rows that are not a multiple of the workgroup's 16,
blocks per row that are not a multiple of the packing group (24 blocks),
weight-row prefixes (forward_rows), awkward activations (a zero block,
outliers, ties, a doubled maximum, subnormal and huge values), the
summation-order known answers of the oracle's tests, the 8B shapes at
decode, and the host's argument errors.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

QT = {"q4_0": hip.GGML_Q4_0, "q8_0": hip.GGML_Q8_0}
NP = {"f32": np.float32, "f16": np.float16}


def weight(ctx, rng, qtype, n, k, d_range=(0.004, 0.012)):
    raw = W.quant_table(rng, n, k, qtype, d_range)
    return raw, ops.QmmWeight.from_raw(ctx, QT[qtype], raw, n, k)


def awkward(rng, m, k, scale=3.0, huge=1e30):
    """qmm/tests.rs:199-208 plus a block of tiny values (their scale is an f32
    subnormal) and a block of huge ones (`huge`, 1e4 where f16 must hold it)."""
    x = (rng.uniform(-1.0, 1.0, (m, k)) * scale).astype(np.float32)
    x[:, :32] = 0.0
    if k >= 64:
        x[:, 32 + 3] = 127.0
        x[:, 32 + 4] = 0.5
        x[:, 32 + 5] = -1.5
    if k >= 96:
        x[:, 64 + 10] = -9.0
        x[:, 64 + 20] = 9.0
    if k >= 160:
        x[:, 96:128] *= np.float32(1e-38)   # subnormal products of the scale
        x[:, 128:160] *= np.float32(huge)
    return x


def want_out(raw, qtype, n, k, x, rows, dtype):
    w = O.qmm(raw, QT[qtype], n, k, x, rows=rows, threads=8)
    return w.astype(np.float16) if dtype == "f16" else w


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("n,k,m", [(10, 512, 7), (3, 256, 1), (130, 512, 41), (9, 1024, 2),
                                   (10, 64, 7), (3, 96, 1), (37, 128, 6), (40, 768, 3),
                                   (17, 4096, 4), (33, 2048, 5), (16, 14336, 1)])
def test_qmm_is_bit_exact(ctx, qtype, dtype, n, k, m):
    rng = np.random.default_rng(n * 31 + k + m)
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, m, k, huge=1e30 if dtype == "f32" else 1e4).astype(NP[dtype])
    got = w.forward(ctx.array(x)).numpy()
    assert_bits_equal(got, want_out(raw, qtype, n, k, x, n, dtype), f"{qtype} {dtype} {n}x{k} m={m}")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_weight_row_prefix(ctx, qtype):
    rng = np.random.default_rng(17)
    for n, k, m, rows in [(10, 512, 3, 7), (600, 256, 2, 450), (64, 768, 5, 1), (100, 128, 1, 99)]:
        raw, w = weight(ctx, rng, qtype, n, k)
        x = awkward(rng, m, k)
        dx = ctx.array(x)
        part = w.forward_rows(dx, rows).numpy()
        assert_bits_equal(part, want_out(raw, qtype, n, k, x, rows, "f32"), f"rows {rows} of {n}")
        assert_bits_equal(part, w.forward(dx).numpy()[:, :rows], "prefix of the whole product")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_a_row_is_bit_identical_alone_and_in_any_batch(ctx, qtype):
    rng = np.random.default_rng(3)
    n, k = 70, 512
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, 17, k)
    alone = [w.forward(ctx.array(x[j:j + 1])).numpy()[0] for j in range(17)]
    for m in (2, 3, 4, 5, 8, 9, 17):
        batch = w.forward(ctx.array(x[:m])).numpy()
        for j in range(m):
            assert_bits_equal(batch[j], alone[j], f"row {j} of a batch of {m}")


def _ones_block_x(d, entries):
    x = np.zeros(32, np.float32)
    x[31] = 127.0 * d
    for e, qv in entries.items():
        x[e] = qv * d
    return x


def _q8_block(d, quants):
    b = np.zeros(34, np.uint8)
    b[:2] = np.array([d], np.float16).view(np.uint8)
    b[2:] = np.asarray(quants, np.int8).view(np.uint8)
    return b


def test_summation_order_known_answers(ctx):
    """The oracle tests' hand-built cases: the lanes sum sequentially over the
    blocks and are reduced by the hsum tree (answers 1.0)."""
    # lanes sequential over blocks, then the tree
    x = np.concatenate([_ones_block_x(1024.0, {0: 64, 16: 64}), _ones_block_x(1.0, {8: 1}),
                        _ones_block_x(1024.0, {0: 64, 16: 64})]).reshape(1, 96)
    w0 = np.zeros(32, np.int8); w0[0] = 64; w0[16] = 64
    w1 = np.zeros(32, np.int8); w1[8] = 1
    w2 = np.zeros(32, np.int8); w2[0] = -64; w2[16] = -64
    raw = np.concatenate([_q8_block(1024.0, w0), _q8_block(1.0, w1), _q8_block(1024.0, w2)])
    w = ops.QmmWeight.from_raw(ctx, hip.GGML_Q8_0, raw, 1, 96)
    assert w.forward(ctx.array(x)).numpy()[0, 0] == 1.0
    # the tree: a[0] + a[8] first
    x = np.concatenate([_ones_block_x(1024.0, {0: 64, 16: 64, 8: 64, 24: 64}),
                        _ones_block_x(1.0, {1: 1})]).reshape(1, 64)
    w0 = np.zeros(32, np.int8); w0[0] = 64; w0[16] = 64; w0[8] = -64; w0[24] = -64
    w1 = np.zeros(32, np.int8); w1[1] = 1
    raw = np.concatenate([_q8_block(1024.0, w0), _q8_block(1.0, w1)])
    w = ops.QmmWeight.from_raw(ctx, hip.GGML_Q8_0, raw, 1, 64)
    assert w.forward(ctx.array(x)).numpy()[0, 0] == 1.0


def test_zero_activations_give_exact_zeros(ctx):
    rng = np.random.default_rng(6)
    for qtype in ("q4_0", "q8_0"):
        _, w = weight(ctx, rng, qtype, 33, 512)
        out = w.forward(ctx.array(np.zeros((4, 512), np.float32))).numpy()
        assert np.all(out == 0.0) and not np.signbit(out).any()


def glu_floor(g, u, act):
    if act != hip.ACT_GELU_TANH:
        return None
    return 2.0 ** -22 * np.abs(0.5 * g.astype(np.float64) * u.astype(np.float64))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("ff,k,m,clamp", [(96, 512, 1, 0.0), (200, 256, 3, 0.0), (48, 768, 5, 0.0),
                                          (64, 1024, 2, 2.0), (1000, 2048, 1, 0.0)])
def test_qmm_glu(ctx, qtype, dtype, act, ff, k, m, clamp):
    rng = np.random.default_rng(ff + k + m + act)
    graw, gw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    uraw, uw = weight(ctx, rng, qtype, ff, k, (0.01, 0.05))
    x = awkward(rng, m, k, 1.0, huge=100.0).astype(NP[dtype])
    got = ops.QmmWeight.glu(gw, uw, ctx.array(x), ops.Glu(act, clamp)).numpy()
    g = O.qmm(graw, QT[qtype], ff, k, x, threads=8)
    u = O.qmm(uraw, QT[qtype], ff, k, x, threads=8)
    want = O.glu(g, u, act, clamp=clamp)
    gc = np.minimum(g, clamp) if clamp > 0 else g
    uc = np.clip(u, -clamp, clamp) if clamp > 0 else u
    if dtype == "f16":
        # the kernel rounds act(g) * u once; the oracle's f16 is that of its f32
        assert_close(got, want.astype(np.float16), floor=glu_floor(gc, uc, act),
                     what=f"glu {qtype} f16")
    else:
        assert_close(got, want, floor=glu_floor(gc, uc, act), what=f"glu {qtype} f32")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("ff,k,m,clamp", [(200, 256, 3, 0.0), (48, 768, 5, 0.0), (64, 1024, 2, 2.0),
                                          (1000, 2048, 4, 0.0)])
def test_qmm_glu_f16_finite(ctx, qtype, act, ff, k, m, clamp):
    """f16 GLU outputs that all stay within f16 range (smaller weight scales
    than test_qmm_glu, whose Q8_0 f16 cases overflow), so the f16 epilogue
    is checked on finite values too."""
    rng = np.random.default_rng(5 * ff + k + m + act)
    graw, gw = weight(ctx, rng, qtype, ff, k, (0.001, 0.004))
    uraw, uw = weight(ctx, rng, qtype, ff, k, (0.001, 0.004))
    x = awkward(rng, m, k, 1.0, huge=1.0).astype(np.float16)
    got = ops.QmmWeight.glu(gw, uw, ctx.array(x), ops.Glu(act, clamp)).numpy()
    g = O.qmm(graw, QT[qtype], ff, k, x, threads=8)
    u = O.qmm(uraw, QT[qtype], ff, k, x, threads=8)
    want = O.glu(g, u, act, clamp=clamp).astype(np.float16)
    assert np.all(np.isfinite(want))
    gc = np.minimum(g, clamp) if clamp > 0 else g
    uc = np.clip(u, -clamp, clamp) if clamp > 0 else u
    assert_close(got, want, floor=glu_floor(gc, uc, act), what=f"glu {qtype} f16 finite")


@pytest.mark.parametrize("qtype,name,n,k", [("q4_0", "ffn_gate", 14336, 4096),
                                            ("q8_0", "ffn_down", 4096, 14336),
                                            ("q4_0", "attn_q", 4096, 4096)])
@pytest.mark.parametrize("m", [1, 4])
def test_llama3_8b_shapes(ctx, qtype, name, n, k, m):
    rng = np.random.default_rng(n + k + m)
    raw, w = weight(ctx, rng, qtype, n, k, (0.001, 0.02))
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = w.forward(ctx.array(x)).numpy()
    assert_bits_equal(got, want_out(raw, qtype, n, k, x, n, "f32"), f"{name} m={m}")


def test_host_rejects_bad_arguments(ctx):
    rng = np.random.default_rng(1)
    raw, w = weight(ctx, rng, "q4_0", 8, 256)
    x = ctx.array(rng.standard_normal((2, 256)).astype(np.float32))
    out = ctx.empty((2, 8), np.float32)
    for rows in (0, 9):
        with pytest.raises(hip.CucaError, match="weight rows"):
            ctx.qmm(w.packed.ptr, hip.GGML_Q4_0, 8, 256, x.ptr, 256, 2, rows, out.ptr, 8, hip.F32)
    with pytest.raises(hip.CucaError, match="Q4_0"):
        ctx.qmm(w.packed.ptr, 3, 8, 256, x.ptr, 256, 2, 8, out.ptr, 8, hip.F32)
    with pytest.raises(hip.CucaError, match="whole number of blocks"):
        ctx.qmm(w.packed.ptr, hip.GGML_Q4_0, 8, 250, x.ptr, 256, 2, 8, out.ptr, 8, hip.F32)
    with pytest.raises(hip.CucaError, match="aligned"):
        ctx.qmm(w.packed.ptr, hip.GGML_Q4_0, 8, 256, x.ptr + 4, 256, 2, 8, out.ptr, 8, hip.F32)
    with pytest.raises(hip.CucaError, match="activations hold"):
        w.forward(ctx.array(np.zeros((2, 128), np.float32)))
    assert ops.QmmWeight.from_raw(ctx, hip.GGML_Q4_0, raw[:-1], 8, 256) is None
    assert ops.QmmWeight.from_raw(ctx, hip.GGML_Q4_0, raw, 8, 250) is None
    # m = 0 is a no-op
    ctx.qmm(w.packed.ptr, hip.GGML_Q4_0, 8, 256, x.ptr, 256, 0, 8, out.ptr, 8, hip.F32)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("m,k", [(1, 32), (2, 4096), (5, 14336), (3, 96)])
def test_q8_acts_is_the_reference_quantisation(ctx, dtype, m, k):
    """cuca_hip_q8_acts = Acts::new (quants and f16-rounded scales, bit for bit)."""
    rng = np.random.default_rng(m * k)
    x = awkward(rng, m, k, huge=1e30 if dtype == "f32" else 1e4).astype(NP[dtype])
    dx = ctx.array(x)
    q, s = ctx.empty((m, k), np.int8), ctx.empty((m, k // 32), np.float32)
    ctx.q8_acts(dx.ptr, k, m, k, hip.dtype_code(NP[dtype]), q.ptr, s.ptr)
    wq, ws = O.q8_acts(x)
    assert np.array_equal(q.numpy(), wq)
    assert_bits_equal(s.numpy(), ws, "act scales")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m", [1, 2])
def test_qmv_two_steps(ctx, qtype, m):
    """q8_acts once, then qmv (plain) and qmv_glu on the same quants."""
    rng = np.random.default_rng(m + 7)
    n, k = 300, 4096
    graw, gw = weight(ctx, rng, qtype, n, k, (0.01, 0.05))
    uraw, uw = weight(ctx, rng, qtype, n, k, (0.01, 0.05))
    x = awkward(rng, m, k, 1.0, huge=100.0)
    dx = ctx.array(x)
    q, s = ctx.empty((m, k), np.int8), ctx.empty((m, k // 32), np.float32)
    ctx.q8_acts(dx.ptr, k, m, k, hip.F32, q.ptr, s.ptr)
    out = ctx.empty((m, n), np.float32)
    ctx.qmv(gw.packed.ptr, QT[qtype], n, k, q.ptr, s.ptr, m, n, out.ptr, n, hip.F32)
    g = O.qmm(graw, QT[qtype], n, k, x)
    assert_bits_equal(out.numpy(), g, "qmv")
    ctx.qmv_glu(gw.packed.ptr, uw.packed.ptr, QT[qtype], n, k, q.ptr, s.ptr, m, hip.ACT_SILU, 0.0, out.ptr, n,
                hip.F32)
    u = O.qmm(uraw, QT[qtype], n, k, x)
    assert_close(out.numpy(), O.glu(g, u, hip.ACT_SILU), what="qmv glu")
    with pytest.raises(hip.CucaError, match="decode GEMV"):
        ctx.qmv(gw.packed.ptr, QT[qtype], n, k, q.ptr, s.ptr, 3, n, out.ptr, n, hip.F32)


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m", [1, 2])
def test_rows_too_long_for_the_decode_gemv_take_the_chunked_kernel(ctx, qtype, m):
    rng = np.random.default_rng(m + 11)
    n, k = 40, 16384 if m == 1 else 14336
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, m, k)
    assert_bits_equal(w.forward(ctx.array(x)).numpy(), want_out(raw, qtype, n, k, x, n, "f32"), f"k={k} m={m}")


@pytest.mark.parametrize("m", [1, 2])
def test_lm_head_on_the_decode_gemv(ctx, m):
    """A vocabulary tall enough (40000 rows) for the many-row routes: two
    rows take the decode GEMV (each wave running several tasks), one row the
    one-row kernel's 8-wave workgroups."""
    rng = np.random.default_rng(m)
    vocab, k = 40000, 512
    raw, w = weight(ctx, rng, "q8_0", vocab, k, (0.01, 0.05))
    x = (rng.standard_normal((m, k)) * 4).astype(np.float32)
    dx = ctx.array(x)
    out = ctx.empty((m, vocab), np.float32)
    for scale, mult, cap in [(1.0, 1.0, 0.0), (3.0, 0.5, 0.0), (1.0, 1.0, 30.0)]:
        ctx.lm_head(w.packed.ptr, hip.GGML_Q8_0, vocab, k, dx.ptr, k, m, vocab, scale, mult, cap, out.ptr,
                    vocab, hip.F32)
        want = O.cap_logits(O.qmm(raw, hip.GGML_Q8_0, vocab, k, x, threads=8), scale, mult, cap)
        if cap == 0.0:
            assert_bits_equal(out.numpy(), want, "lm head")
        else:
            assert np.all(np.abs(out.numpy() - want) <= 2.0 ** -22 * cap + 1e-6 * np.abs(want))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("glu", [False, True])
def test_decode_gemv_waves_that_run_several_tasks(ctx, qtype, glu):
    """40000 rows at one activation row: the one-row kernel's 8-wave
    workgroups (plain and GLU), the LM head's route."""
    rng = np.random.default_rng(40000 + glu)
    n, k = 40000, 256
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, 1, k, 1.0, huge=100.0)
    dx = ctx.array(x)
    if glu:
        uraw, uw = weight(ctx, rng, qtype, n, k)
        got = ops.QmmWeight.glu(w, uw, dx, ops.Glu(hip.ACT_SILU)).numpy()
        g = O.qmm(raw, QT[qtype], n, k, x, threads=8)
        u = O.qmm(uraw, QT[qtype], n, k, x, threads=8)
        assert_close(got, O.glu(g, u, hip.ACT_SILU), what="several tasks, glu")
    else:
        assert_bits_equal(w.forward(dx).numpy(), want_out(raw, qtype, n, k, x, n, "f32"), "several tasks")


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_decode_gemv_streams_chunks_of_tasks(ctx, qtype):
    """600000 rows of 64 values: more than 32 four-row tasks per wave of the
    persistent grid, so a wave streams several chunks of tasks (sums staged
    in LDS, written per chunk); through the quantised rows (cuca_hip_qmv)
    and through qmm's routing (the rows of x)."""
    rng = np.random.default_rng(600000)
    n, k = 600000, 64
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, 2, k, 1.0, huge=100.0)
    dx = ctx.array(x)
    want = want_out(raw, qtype, n, k, x, n, "f32")
    assert_bits_equal(w.forward(dx).numpy(), want, "streamed chunks, rows of x")
    q, s = ctx.empty((2, k), np.int8), ctx.empty((2, k // 32), np.float32)
    ctx.q8_acts(dx.ptr, k, 2, k, hip.F32, q.ptr, s.ptr)
    out = ctx.empty((2, n), np.float32)
    ctx.qmv(w.packed.ptr, QT[qtype], n, k, q.ptr, s.ptr, 2, n, out.ptr, n, hip.F32)
    assert_bits_equal(out.numpy(), want, "streamed chunks, quantised rows")


# ---------------------------------------------------------------------------
# the Q|K|V projection with RoPE and the paged K/V store in its epilogue
# (cuca_hip_qmm_rope_store_kv): the bits of qmm followed by rope_store_kv
# ---------------------------------------------------------------------------

def qkv_fused_vs_unfused(ctx, rng, qtype, dtype, nq, nk, d, k, m, n_dims=None, bad_row=None):
    n_dims = d if n_dims is None else n_dims
    n = (nq + 2 * nk) * d
    raw, w = weight(ctx, rng, qtype, n, k)
    x = awkward(rng, m, k, huge=1e30 if dtype == "f32" else 1e4).astype(NP[dtype])
    n_blocks = 8 + m
    cos, sin = hip.rope_tables(hip.ROPE_NORM, n_dims, 5e5, 8192)
    pos = rng.integers(0, 8192, m).astype(np.int32)
    slots = rng.permutation(n_blocks * 16)[:m].astype(np.int32)
    if bad_row is not None:
        slots[bad_row] = n_blocks * 16 + 3            # outside the pool
    dcos, dsin, dpos, dslots = ctx.array(cos), ctx.array(sin), ctx.array(pos), ctx.array(slots)
    dx = ctx.array(x)
    init = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    # unfused: qmm into a [m, n] Q|K|V buffer, then rope_store_kv reading it in place
    pool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
    pool.k.upload(init)
    pool.v.upload(init)
    qkv = w.forward(dx)
    es = np.dtype(NP[dtype]).itemsize
    ctx.rope_store_kv(qkv.ptr, n, qkv.ptr + nq * d * es, n, qkv.ptr + (nq + nk) * d * es, n, m, nq, nk, d,
                      n_dims, hip.ROPE_NORM, dcos.ptr, dsin.ptr, 8192, dpos.ptr, None, None, 0, 1e-6,
                      pool.k.ptr, pool.v.ptr, n_blocks, dslots.ptr, hip.dtype_code(NP[dtype]))
    if bad_row is not None:
        with pytest.raises(hip.CucaError, match="K/V slot"):
            ctx.check_device()
    ctx.check_device()
    want_q, want_k, want_v = qkv.numpy()[:, :nq * d], pool.k.numpy(), pool.v.numpy()
    # fused
    fpool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
    fpool.k.upload(init)
    fpool.v.upload(init)
    q_out = ctx.empty((m, nq * d), NP[dtype])
    ctx.qmm_rope_store_kv(w.packed.ptr, QT[qtype], k, dx.ptr, k, m, nq, nk, d, n_dims, hip.ROPE_NORM,
                          dcos.ptr, dsin.ptr, 8192, dpos.ptr, q_out.ptr, nq * d, fpool.k.ptr, fpool.v.ptr,
                          n_blocks, dslots.ptr, hip.dtype_code(NP[dtype]))
    if bad_row is not None:
        with pytest.raises(hip.CucaError, match="K/V slot"):
            ctx.check_device()
    ctx.check_device()
    assert_bits_equal(q_out.numpy(), want_q, "fused q")
    assert_bits_equal(fpool.k.numpy(), want_k, "fused pool k")
    assert_bits_equal(fpool.v.numpy(), want_v, "fused pool v")
    return raw, x, pos, slots, cos, sin, q_out.numpy(), fpool


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d,k,m", [(32, 8, 128, 4096, 1), (32, 8, 128, 4096, 2), (32, 8, 128, 4096, 5),
                                         (4, 2, 64, 512, 3), (6, 2, 16, 256, 1)])
def test_qkv_rope_store_fused_is_qmm_then_rope_store(ctx, qtype, dtype, nq, nk, d, k, m):
    rng = np.random.default_rng(nq + nk + d + k + m)
    qkv_fused_vs_unfused(ctx, rng, qtype, dtype, nq, nk, d, k, m)


def test_qkv_rope_store_fused_partial_rotary_bad_slot_and_oracle(ctx):
    rng = np.random.default_rng(77)
    # partial rotary: values past n_dims pass through
    qkv_fused_vs_unfused(ctx, rng, "q4_0", "f32", 4, 2, 64, 512, 2, n_dims=32)
    # a bad slot: the row keeps Q unrotated and stores no K/V, reported
    qkv_fused_vs_unfused(ctx, rng, "q8_0", "f32", 4, 2, 32, 256, 3, bad_row=1)
    # against the oracle directly: qmm, then store_kv
    nq, nk, d, k, m = 4, 2, 32, 256, 3
    raw, x, pos, slots, cos, sin, got_q, fpool = qkv_fused_vs_unfused(ctx, rng, "q4_0", "f32", nq, nk, d, k, m)
    n = (nq + 2 * nk) * d
    y = O.qmm(raw, hip.GGML_Q4_0, n, k, x, rows=n, threads=4)
    wq = O.rope(y[:, :nq * d].reshape(m, nq, d), cos, sin, pos, O.ROPE_NORM)
    assert_bits_equal(got_q.reshape(m, nq, d), wq, "oracle q")
    wk = O.rope(y[:, nq * d:(nq + nk) * d].reshape(m, nk, d), cos, sin, pos, O.ROPE_NORM)
    pk = fpool.k.numpy()
    for j in range(m):
        b, r = slots[j] // 16, slots[j] % 16
        assert_bits_equal(pk[b, :, r], wk[j], "oracle pool k")
    with pytest.raises(hip.CucaError, match="only NORM"):
        ctx.qmm_rope_store_kv(fpool.k.ptr, hip.GGML_Q4_0, k, fpool.k.ptr, k, m, nq, nk, d, d, hip.ROPE_NEOX,
                              fpool.k.ptr, fpool.k.ptr, 8192, fpool.k.ptr, fpool.k.ptr, nq * d, fpool.k.ptr,
                              fpool.v.ptr, 8, fpool.k.ptr, hip.F32)
