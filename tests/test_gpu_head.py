"""The end of a step on the GPU (cuca_hip_lm_head, cuca_hip_argmax,
cuca_hip_top_k) against the oracle, through the C ABI.

Bars:
- lm_head without a soft-cap: bit-exact (the qmm bits, then candle's affine
  multiplies); with a soft-cap: |got - want| <= 2^-22 * cap + 1e-6 |want|
  (tanh is the device's, within 2 ulp of the reference's libm tanhf);
- argmax: the same id as greedy (first maximum), rows with ties, NaN and
  -inf included;
- top_k: the same candidates, bit for bit (the scaled logits) and id for
  id, in the same order as select_top_k, for k from 1 to 1024, temperatures
  other than 1, many equal logits, masked entries and rows with fewer finite
  logits than k;
- device top-k + the library's host finish draw the same ids as the
  reference's sample on the whole row, for 64 seeds.
"""
import ctypes

import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("scale,mult,cap", [(1.0, 1.0, 0.0), (3.0, 1.0, 0.0), (1.0, 0.25, 0.0),
                                            (1.0, 1.0, 30.0), (2.0, 0.5, 15.0)])
def test_lm_head(ctx, qtype, scale, mult, cap):
    rng = np.random.default_rng(int(scale * 10 + mult * 100 + cap))
    vocab, k, m = 1000, 512, 3
    raw = W.quant_table(rng, vocab, k, qtype, (0.01, 0.05))
    w = ops.QmmWeight.from_raw(ctx, W.GGML_ID[qtype], raw, vocab, k)
    x = (rng.standard_normal((m, k)) * 4).astype(np.float32)
    dx = ctx.array(x)
    out = ctx.empty((m, vocab), np.float32)
    ctx.lm_head(w.packed.ptr, W.GGML_ID[qtype], vocab, k, dx.ptr, k, m, vocab, scale, mult, cap,
                out.ptr, vocab, hip.F32)
    got = out.numpy()
    want = O.cap_logits(O.qmm(raw, W.GGML_ID[qtype], vocab, k, x), scale, mult, cap)
    if cap == 0.0:
        assert_bits_equal(got, want, "lm head")
    else:
        assert np.all(np.abs(got - want) <= 2.0 ** -22 * cap + 1e-6 * np.abs(want))
        assert np.all(np.abs(got) <= cap)


def test_lm_head_rows_prefix_and_errors(ctx):
    rng = np.random.default_rng(1)
    raw = W.quant_table(rng, 300, 256, "q8_0", (0.01, 0.05))
    w = ops.QmmWeight.from_raw(ctx, hip.GGML_Q8_0, raw, 300, 256)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    dx = ctx.array(x)
    out = ctx.empty((2, 100), np.float32)
    ctx.lm_head(w.packed.ptr, hip.GGML_Q8_0, 300, 256, dx.ptr, 256, 2, 100, 1.0, 1.0, 0.0, out.ptr, 100,
                hip.F32)
    assert_bits_equal(out.numpy(), O.qmm(raw, hip.GGML_Q8_0, 300, 256, x, rows=100), "head_rows")
    with pytest.raises(hip.CucaError, match="soft-cap"):
        ctx.lm_head(w.packed.ptr, hip.GGML_Q8_0, 300, 256, dx.ptr, 256, 2, 100, 0.0, 1.0, 0.0, out.ptr,
                    100, hip.F32)


def logits_rows(rng, rows, vocab, kind):
    if kind == "normal":
        x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    elif kind == "ties":
        x = np.floor(rng.uniform(0, 16, (rows, vocab))).astype(np.float32)
    else:  # masked: mostly -inf, a few values, NaNs
        x = np.full((rows, vocab), -np.inf, np.float32)
        for r in range(rows):
            idx = rng.choice(vocab, min(vocab - 3, 20 + r), replace=False)
            x[r, idx] = rng.standard_normal(idx.size).astype(np.float32)
            x[r, rng.choice(vocab, 3, replace=False)] = np.nan
    return x


@pytest.mark.parametrize("vocab", [7, 1000, 128256, 151936, 256000])
@pytest.mark.parametrize("kind", ["normal", "ties", "masked"])
def test_argmax(ctx, vocab, kind):
    rng = np.random.default_rng(vocab + len(kind))
    rows = 4
    x = logits_rows(rng, rows, vocab, kind)
    if kind == "normal":
        x[1, :] = -np.inf            # no value above -inf: id 0
        x[2, vocab // 2:] = x[2].max() + 1.0   # ties at the maximum: the first
    ids = ctx.empty((rows,), np.uint32)
    dx = ctx.array(x)
    ctx.argmax(dx.ptr, vocab, rows, vocab, hip.F32, ids.ptr)
    assert ids.numpy().tolist() == [O.greedy(x[r]) for r in range(rows)]
    x16 = x.astype(np.float16)
    dx16 = ctx.array(x16)
    ctx.argmax(dx16.ptr, vocab, rows, vocab, hip.F16, ids.ptr)
    assert ids.numpy().tolist() == [O.greedy(x16[r].astype(np.float32)) for r in range(rows)]


@pytest.mark.parametrize("vocab,k", [(1000, 1), (1000, 2), (1000, 40), (128256, 40), (151936, 333),
                                     (256000, 1024), (5000, 1024), (100, 1000)])
@pytest.mark.parametrize("kind", ["normal", "ties", "masked"])
@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_top_k(ctx, vocab, k, kind, temperature):
    rng = np.random.default_rng(vocab + k + len(kind))
    rows = 3
    x = logits_rows(rng, rows, vocab, kind)
    dx = ctx.array(x)
    ol, oi, oc = ctx.empty((rows, k), np.float32), ctx.empty((rows, k), np.uint32), ctx.empty((rows,), np.int32)
    ctx.top_k(dx.ptr, vocab, rows, vocab, hip.F32, k, temperature, ol.ptr, oi.ptr, oc.ptr)
    gl, gi, gc = ol.numpy(), oi.numpy(), oc.numpy()
    for r in range(rows):
        wl, wi = O.select_top_k(x[r], temperature, k)
        assert gc[r] == wl.size, (r, gc[r], wl.size)
        assert gi[r, :gc[r]].tolist() == wi.tolist()
        assert_bits_equal(gl[r, :gc[r]], wl, f"top-k logits row {r}")


@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_many_rows_take_each_row_whole(ctx, kind):
    """600 rows: one workgroup per row, no slices and no merge launch; a
    32000-value row fills the workgroup's LDS several times over (rounds of
    selection that carry the kept candidates forward)."""
    rng = np.random.default_rng(600 + len(kind))
    rows, vocab, k = 600, 32000, 50
    x = logits_rows(rng, rows, vocab, kind)
    x[7, :] = -np.inf
    x[8, :200] = np.nan
    dx = ctx.array(x)
    ol, oi, oc = ctx.empty((rows, k), np.float32), ctx.empty((rows, k), np.uint32), ctx.empty((rows,), np.int32)
    ctx.top_k(dx.ptr, vocab, rows, vocab, hip.F32, k, 0.9, ol.ptr, oi.ptr, oc.ptr)
    ids = ctx.empty((rows,), np.uint32)
    ctx.argmax(dx.ptr, vocab, rows, vocab, hip.F32, ids.ptr)
    gl, gi, gc, ga = ol.numpy(), oi.numpy(), oc.numpy(), ids.numpy()
    for r in range(rows):
        wl, wi = O.select_top_k(x[r], 0.9, k)
        assert gc[r] == wl.size, (r, gc[r], wl.size)
        assert gi[r, :gc[r]].tolist() == wi.tolist(), r
        assert_bits_equal(gl[r, :gc[r]], wl, f"top-k logits row {r}")
        assert int(ga[r]) == O.greedy(x[r]), r


def test_device_top_k_then_host_finish_is_the_reference_sample(ctx):
    rng = np.random.default_rng(12)
    vocab, rows = 128256, 2
    x = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    dx = ctx.array(x)
    for temperature, top_k, top_p in [(0.8, 40, 0.95), (1.0, 5, 1.0), (1.2, 100, 0.5)]:
        ol, oi, oc = ctx.empty((rows, top_k), np.float32), ctx.empty((rows, top_k), np.uint32), \
            ctx.empty((rows,), np.int32)
        ctx.top_k(dx.ptr, vocab, rows, vocab, hip.F32, top_k, temperature, ol.ptr, oi.ptr, oc.ptr)
        ids = ctx.empty((rows,), np.uint32)
        ctx.argmax(dx.ptr, vocab, rows, vocab, hip.F32, ids.ptr)
        gl, gi, gc, fb = ol.numpy(), oi.numpy(), oc.numpy(), ids.numpy()
        for r in range(rows):
            for seed in range(64):
                want = O.sample(x[r], temperature, top_k, top_p, O.SplitMix64(seed))
                got = hip.sample_candidates(gl[r, :gc[r]], gi[r, :gc[r]], top_p, int(fb[r]),
                                            ctypes.c_uint64(seed))
                assert got == want, (temperature, top_k, top_p, r, seed)


def test_pick_errors(ctx):
    x = ctx.array(np.zeros((1, 10), np.float32))
    o = ctx.empty((1, 2000), np.float32)
    i = ctx.empty((1, 2000), np.uint32)
    c = ctx.empty((1,), np.int32)
    with pytest.raises(hip.CucaError, match="1..1024"):
        ctx.top_k(x.ptr, 10, 1, 10, hip.F32, 2000, 1.0, o.ptr, i.ptr, c.ptr)
    with pytest.raises(hip.CucaError, match="temperature"):
        ctx.top_k(x.ptr, 10, 1, 10, hip.F32, 5, 0.0, o.ptr, i.ptr, c.ptr)
    with pytest.raises(hip.CucaError, match="logits shape"):
        ctx.argmax(x.ptr, 5, 1, 10, hip.F32, i.ptr)


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m,cap", [(1, 0.0), (3, 0.0), (2, 30.0)])
def test_lm_head_indexed_is_the_full_heads_columns(ctx, qtype, m, cap):
    """head_indexed (cpu.rs:2603-2606, QMatMul::forward_indexed qmm.rs:1818-1843):
    the logits of chosen vocabulary ids, any order and repeats, bit for bit
    the full head's columns (the same kernel per weight row)."""
    rng = np.random.default_rng(m + int(cap))
    vocab, k = 4100, 1024
    T = W.GGML_ID[qtype]
    raw = W.quant_table(rng, vocab, k, qtype, (0.01, 0.05))
    w = ops.QmmWeight.from_raw(ctx, T, raw, vocab, k)
    x = (rng.standard_normal((m, k)) * 4).astype(np.float32)
    dx = ctx.array(x)
    full = ctx.empty((m, vocab), np.float32)
    ctx.lm_head(w.packed.ptr, T, vocab, k, dx.ptr, k, m, vocab, 1.0, 1.0, cap, full.ptr, vocab, hip.F32)
    ids = np.concatenate([[vocab - 1, 0, 17, 17], rng.integers(0, vocab, 300)]).astype(np.uint32)
    n = ids.size
    wsb = hip.lm_head_indexed_workspace(T, k, n)
    assert wsb == n * hip.qweight_bytes(T, 1, k)
    ws = ctx.empty((wsb,), np.uint8)
    out = ctx.empty((m, n + 3), np.float32)
    ctx.lm_head_indexed(w.packed.ptr, T, vocab, k, dx.ptr, k, m, ctx.array(ids).ptr, n, 1.0, 1.0, cap, ws.ptr,
                        wsb, out.ptr, n + 3, hip.F32)
    ctx.check_device()
    assert_bits_equal(out.numpy()[:, :n], full.numpy()[:, ids], "indexed head")
    if cap == 0.0:
        want = O.qmm(raw, T, vocab, k, x)[:, ids]
        assert_bits_equal(out.numpy()[:, :n], want, "indexed head vs oracle")


def test_lm_head_indexed_errors(ctx):
    rng = np.random.default_rng(3)
    vocab, k = 64, 256
    raw = W.quant_table(rng, vocab, k, "q8_0", (0.01, 0.05))
    w = ops.QmmWeight.from_raw(ctx, hip.GGML_Q8_0, raw, vocab, k)
    dx = ctx.array(rng.standard_normal((1, k)).astype(np.float32))
    ids = ctx.array(np.array([3, 64, 5], np.uint32))
    wsb = hip.lm_head_indexed_workspace(hip.GGML_Q8_0, k, 3)
    ws = ctx.empty((wsb,), np.uint8)
    out = ctx.empty((1, 3), np.float32)
    with pytest.raises(hip.CucaError, match="workspace of"):
        ctx.lm_head_indexed(w.packed.ptr, hip.GGML_Q8_0, vocab, k, dx.ptr, k, 1, ids.ptr, 3, 1.0, 1.0, 0.0, ws.ptr,
                            wsb - 16, out.ptr, 3, hip.F32)
    ctx.lm_head_indexed(w.packed.ptr, hip.GGML_Q8_0, vocab, k, dx.ptr, k, 1, ids.ptr, 3, 1.0, 1.0, 0.0, ws.ptr,
                        wsb, out.ptr, 3, hip.F32)
    with pytest.raises(hip.CucaError, match="weight row 64 out of range"):
        ctx.check_device()
    assert out.numpy()[0, 1] == 0.0
