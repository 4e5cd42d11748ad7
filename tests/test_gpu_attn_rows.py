"""Attention of many rows of one sequence over its paged cache
(cuca_hip_attend_rows, cuca_hip_attend_latent_rows) on the GPU, against the
oracle's restatement of attend_paged_rows (cpu/paged_attn.rs:177-309), which
tests/test_oracle_attn.py pins to f64 attention over the gathered keys.

Bar (as the decode kernel's): |got - want| <= 1e-5 |want| + 1e-5 max|v|
(f32), 2 f16 ulps + the same floor (f16), max|v| the largest value magnitude
of the row's range in that KV head.  The latent form's oracle is the same
function with the key pool as the value pool, its first v_width columns
(each output column depends on that value column only).

Covers: causal prefill chunks that continue a cache (rows at positions
start..start+t-1, row i over lo..start+i+1), a window floor with released
blocks before it, partial tiles of 16 rows, the configs' head layouts
(matrix-core kernels: head_dim 64/128/256, groups 1-8, f32 and f16), shapes
that take the generic kernel (head_dim 48, group 3, a q row stride the
matrix-core loads cannot take), a row's bits alone and in its chunk, bad
ranges and blocks (zero rows, reported; a missing block at the end of
the kernel's first 64-entry table window), the latent form (head_dim 576,
v_width 512 of DeepSeek-style caches, and a small one), and host checks.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.float16}


def chunk(rng, t, start, n_blocks, width, window=None):
    """A sequence of start + t positions over scrambled blocks, the chunk's
    rows at positions start..start+t-1, causal ranges (a window floor:
    positions before hi - window dropped, their blocks released)."""
    nb = (start + t + 15) // 16
    table = np.full(width, O.NO_BLOCK, np.uint32)
    table[:nb] = rng.choice(n_blocks, nb, replace=False)
    hi = start + np.arange(t) + 1
    lo = np.zeros(t, np.int64) if window is None else np.maximum(hi - window, 0)
    if window is not None:
        table[:int(lo.min()) // 16] = O.NO_BLOCK
    return table, np.stack([lo, hi], 1).astype(np.int32)


def floor_of(table, ranges, pool_v, n_head, v_width=None):
    rows = len(ranges)
    n_kv, d = pool_v.shape[1], pool_v.shape[3]
    vw = d if v_width is None else v_width
    f = np.zeros((rows, n_head, vw))
    for r in range(rows):
        lo, hi = ranges[r]
        vals = O.gather(table, lo, hi, pool_v)[..., :vw].astype(np.float64)
        f[r] = 1e-5 * np.repeat(np.abs(vals).max(axis=(1, 2)), n_head // n_kv)[:, None]
    return f


def run_rows(ctx, q, pk, pv, table, ranges, n_head, scale, q_ld=None):
    rows, _, d = q.shape
    n_blocks, n_kv = pk.shape[0], pk.shape[1]
    q_ld = n_head * d if q_ld is None else q_ld
    qpad = np.zeros((rows, q_ld), q.dtype)
    qpad[:, :n_head * d] = q.reshape(rows, -1)
    dq, dk, dv = ctx.array(qpad), ctx.array(pk), ctx.array(pv)
    dt, dr = ctx.array(table.astype(np.uint32)), ctx.array(ranges.astype(np.int32))
    out = ctx.empty((rows, n_head, d), q.dtype)
    ctx.attend_rows(dq.ptr, q_ld, dk.ptr, dv.ptr, n_blocks, dt.ptr, len(table), dr.ptr, rows, n_head, n_kv, d,
                    scale, out.ptr, n_head * d, hip.dtype_code(q.dtype))
    ctx.check_device()
    return out.numpy()


def want_rows(q, pk, pv, table, ranges, scale):
    tables = np.repeat(table[None], len(ranges), 0)
    return O.paged_attention(q, tables, ranges, pk, pv, scale, threads=8)


def check(ctx, q, pk, pv, table, ranges, n_head, scale, q_ld=None):
    got = run_rows(ctx, q, pk, pv, table, ranges, n_head, scale, q_ld)
    want = want_rows(q, pk, pv, table, ranges, scale)
    assert_close(got, want, floor=floor_of(table, ranges, pv, n_head), what="attend_rows")
    return got


@pytest.mark.parametrize("cfg_name,dtype", [("A", "f32"), ("B", "f32"), ("C", "f16"), ("C", "f32"),
                                            ("D", "f32"), ("D", "f16"), ("E", "f32"), ("E", "f16")])
@pytest.mark.parametrize("t,start,window", [(37, 0, None), (64, 50, None), (20, 300, 100)])
def test_configs_causal_chunks(ctx, cfg_name, dtype, t, start, window):
    cfg = W.CONFIGS[cfg_name]
    rng = np.random.default_rng(cfg["seed"] + t + start)
    nq, nk, d = cfg["nq"], cfg["nk"], cfg["head_dim"]
    n_blocks = 64
    table, ranges = chunk(rng, t, start, n_blocks, 40, window)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = (2.0 * rng.standard_normal((t, nq, d))).astype(NP[dtype])
    check(ctx, q, pk, pv, table, ranges, nq, 1.0 / np.sqrt(d))


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d,q_extra", [(6, 2, 48, 0), (3, 1, 64, 0), (4, 2, 64, 2), (2, 2, 32, 0)])
def test_generic_kernel_shapes(ctx, dtype, nq, nk, d, q_extra):
    """head_dim 48 and 32, a group of 3, and (q_extra) a q row stride of
    n_head * d + 2 elements, whose rows the matrix-core kernel's 8-byte (f16)
    query loads cannot take: the generic kernel."""
    rng = np.random.default_rng(nq * 100 + d + q_extra)
    n_blocks = 24
    table, ranges = chunk(rng, 29, 40, n_blocks, 8)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = rng.standard_normal((29, nq, d)).astype(NP[dtype])
    check(ctx, q, pk, pv, table, ranges, nq, 0.3, q_ld=nq * d + q_extra)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_a_row_is_bit_identical_alone_and_in_its_chunk(ctx, dtype):
    """attend_paged_rows' property: a row's result depends only on its query,
    table and range (cpu/paged_attn.rs:9-13)."""
    rng = np.random.default_rng(12)
    nq, nk, d, n_blocks = 32, 8, 128, 48
    table, ranges = chunk(rng, 45, 100, n_blocks, 12)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = rng.standard_normal((45, nq, d)).astype(NP[dtype])
    all_rows = run_rows(ctx, q, pk, pv, table, ranges, nq, 0.1)
    for r in (0, 7, 16, 44):
        one = run_rows(ctx, q[r:r + 1], pk, pv, table, ranges[r:r + 1], nq, 0.1)
        assert_bits_equal(one[0], all_rows[r], f"row {r}")


@pytest.mark.parametrize("nq,nk,d", [(8, 2, 128), (6, 2, 48)])
def test_bad_ranges_and_blocks_give_zero_rows_and_are_reported(ctx, nq, nk, d):
    rng = np.random.default_rng(13)
    n_blocks = 8
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    q = rng.standard_normal((20, nq, d)).astype(np.float32)
    table = np.array([3, 1, 9, 0], np.uint32)   # block 9 is outside the pool of 8
    ranges = np.array([[0, 5 + r] for r in range(20)], np.int32)
    ranges[4] = (7, 7)                          # empty
    with pytest.raises(hip.CucaError, match="attention row 4: empty key range"):
        run_rows(ctx, q, pk, pk, table, ranges, nq, 0.1)
    ranges[4] = (0, 9)
    ranges[17] = (10, 40)                       # reaches block 2 (id 9)
    with pytest.raises(hip.CucaError, match="attention row 17: position 32 has no K/V block"):
        run_rows(ctx, q, pk, pk, table, ranges, nq, 0.1)
    # the same call again, to read its output (the raise reset the status)
    dq, dk = ctx.array(q), ctx.array(pk)
    dt, dr = ctx.array(table), ctx.array(ranges)
    out = ctx.empty((20, nq, d), np.float32)
    ctx.attend_rows(dq.ptr, nq * d, dk.ptr, dk.ptr, n_blocks, dt.ptr, 4, dr.ptr, 20, nq, nk, d, 0.1, out.ptr,
                    nq * d, hip.F32)
    with pytest.raises(hip.CucaError):
        ctx.check_device()
    got = out.numpy()
    assert not np.any(got[17]), "row with a missing block is not zero"
    good = [r for r in range(20) if r != 17]
    want = want_rows(q[good], pk, pk, table, ranges[good], 0.1)
    assert_close(got[good], want, floor=floor_of(table, ranges[good], pk, nq), what="good rows")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_a_missing_block_past_the_first_table_window_is_reported(ctx, dtype):
    """Rows over more than 64 blocks (the kernel holds the table 64 entries
    at a time): block 63, the last of the first window, is outside the pool.
    The rows whose range meets it are zero and reported; the rows of the same
    workgroup whose range starts after it match the oracle."""
    rng = np.random.default_rng(21)
    nq, nk, d, n_blocks = 32, 8, 128, 150
    table = rng.choice(n_blocks, 130, replace=False).astype(np.uint32)
    table[63] = 200                                  # outside the pool of 150
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = rng.standard_normal((32, nq, d)).astype(NP[dtype])
    pos = 1100 + np.arange(32)
    ranges = np.stack([np.where(np.arange(32) < 16, 0, 1024), pos + 1], 1).astype(np.int32)
    dq, dk, dv = ctx.array(q.reshape(32, -1)), ctx.array(pk), ctx.array(pv)
    dt, dr = ctx.array(table), ctx.array(ranges)
    out = ctx.empty((32, nq, d), NP[dtype])
    ctx.attend_rows(dq.ptr, nq * d, dk.ptr, dv.ptr, n_blocks, dt.ptr, len(table), dr.ptr, 32, nq, nk, d, 0.1,
                    out.ptr, nq * d, hip.dtype_code(NP[dtype]))
    with pytest.raises(hip.CucaError, match=r"attention row \d+: position 1008 has no K/V block"):
        ctx.check_device()
    got = out.numpy()
    assert not np.any(got[:16]), "rows over the missing block are not zero"
    want = want_rows(q[16:], pk, pv, table, ranges[16:], 0.1)
    assert_close(got[16:], want, floor=floor_of(table, ranges[16:], pv, nq), what="rows after the block")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nh,d,vw,t", [(16, 576, 512, 21), (4, 80, 64, 33)])
def test_latent_rows(ctx, dtype, nh, d, vw, t):
    """The latent form (attend_latent_rows): one KV head whose rows' first
    v_width columns are the values; out [t, n_head, v_width]."""
    rng = np.random.default_rng(d + vw)
    n_blocks = 16
    table, ranges = chunk(rng, t, 30, n_blocks, 6)
    pool = rng.standard_normal((n_blocks, 1, 16, d)).astype(NP[dtype])
    q = (0.2 * rng.standard_normal((t, nh, d))).astype(NP[dtype])
    dq, dp = ctx.array(q), ctx.array(pool)
    dt, dr = ctx.array(table), ctx.array(ranges)
    out = ctx.empty((t, nh, vw), q.dtype)
    ctx.attend_latent_rows(dq.ptr, nh * d, dp.ptr, n_blocks, dt.ptr, len(table), dr.ptr, t, nh, d, vw, 0.05,
                           out.ptr, nh * vw, hip.dtype_code(q.dtype))
    ctx.check_device()
    want = want_rows(q, pool, pool, table, ranges, 0.05)[..., :vw]
    assert_close(out.numpy(), want, floor=floor_of(table, ranges, pool, nh, vw), what="latent")


def test_host_checks(ctx):
    pool = ops.KvPool(ctx, 4, 2, 64, np.float32)
    q = ctx.array(np.zeros((3, 4, 64), np.float32))
    tab = ctx.array(np.zeros(2, np.uint32))
    rng = ctx.array(np.array([[0, 5]] * 3, np.int32))
    out = ctx.empty((3, 4, 64), np.float32)
    with pytest.raises(hip.CucaError, match="query shape mismatch"):
        ctx.attend_rows(q.ptr, 256, pool.k.ptr, pool.v.ptr, 4, tab.ptr, 2, rng.ptr, 3, 4, 3, 64, 0.1, out.ptr,
                        256, hip.F32)
    with pytest.raises(hip.CucaError, match="null pointer"):
        ctx.attend_rows(q.ptr, 256, pool.k.ptr, None, 4, tab.ptr, 2, rng.ptr, 3, 4, 2, 64, 0.1, out.ptr, 256,
                        hip.F32)
    with pytest.raises(hip.CucaError, match="out row stride"):
        ctx.attend_rows(q.ptr, 256, pool.k.ptr, pool.v.ptr, 4, tab.ptr, 2, rng.ptr, 3, 4, 2, 64, 0.1, out.ptr,
                        255, hip.F32)
    for vw in (0, 65):
        with pytest.raises(hip.CucaError, match="bad latent value width"):
            ctx.attend_latent_rows(q.ptr, 256, pool.k.ptr, 4, tab.ptr, 2, rng.ptr, 3, 4, 64, vw, 0.1, out.ptr,
                                   256, hip.F32)
    # rows 0: nothing to do
    ctx.attend_rows(q.ptr, 256, pool.k.ptr, pool.v.ptr, 4, tab.ptr, 2, rng.ptr, 0, 4, 2, 64, 0.1, out.ptr, 256,
                    hip.F32)


def test_the_pool_method_matches_the_raw_call(ctx):
    rng = np.random.default_rng(14)
    nq, nk, d, n_blocks = 8, 2, 64, 10
    table, ranges = chunk(rng, 18, 20, n_blocks, 4)
    pool = ops.KvPool(ctx, n_blocks, nk, d, np.float16)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float16)
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float16)
    pool.k.upload(pk)
    pool.v.upload(pv)
    q = rng.standard_normal((18, nq, d)).astype(np.float16)
    got = pool.attend_rows(ctx.array(q), ctx.array(table), ctx.array(ranges), nq, 0.125).numpy()
    ctx.check_device()
    assert_bits_equal(got, run_rows(ctx, q, pk, pv, table, ranges, nq, 0.125), "pool method")
