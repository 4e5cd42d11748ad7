"""cuca_hip_paged_decode_noalloc through the C ABI against cuca_hip_paged_decode.

The allocation-free variant runs the same kernels over the library's
per-device scratch array instead of a caller's workspace, so its output must
be the workspace entry point's bits: on two calls in a row (the second with
fewer rows, shorter ranges and another table width, over the scratch the
first call left behind), in f32 and f16.  The workspace of the reference
call is filled with NaN first, so neither side can lean on zeroed memory.
A call whose partials would exceed the scratch is refused on the host.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from helpers import assert_bits_equal
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.float16}


def batch(rng, lengths, n_blocks, width):
    tables = np.full((len(lengths), width), O.NO_BLOCK, np.uint32)
    ranges = np.zeros((len(lengths), 2), np.int32)
    for r, hi in enumerate(lengths):
        nb = (hi + 15) // 16
        tables[r, :nb] = rng.choice(n_blocks, nb, replace=False)
        lo = 0 if r % 3 else max(0, hi - 100)
        tables[r, :lo // 16] = O.NO_BLOCK
        ranges[r] = (lo, hi)
    return tables, ranges


def both(ctx, pool, q, tables, ranges, n_head, scale):
    """(workspace entry point, allocation-free entry point) outputs."""
    rows, _, d = q.shape
    dq, dt, dr = ctx.array(q), ctx.array(tables), ctx.array(ranges)
    need = hip.paged_decode_workspace(rows, n_head, d, tables.shape[1])
    ws = ctx.array(np.full(max(need // 4, 4), np.nan, np.float32))
    want = pool.decode(dq, dt, dr, n_head, scale, workspace=ws).numpy()
    ctx.check_device()
    out = ctx.array(np.full((rows, n_head, d), np.nan, q.dtype))
    got = pool.decode_noalloc(dq, dt, dr, n_head, scale, out=out).numpy()
    ctx.check_device()
    return want, got


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d", [(32, 8, 128), (32, 4, 128), (16, 8, 256), (6, 2, 40)])
def test_noalloc_matches_the_workspace_entry_point_twice(ctx, dtype, nq, nk, d):
    rng = np.random.default_rng(nq * 1000 + nk * 10 + d)
    n_blocks = 160
    pool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
    pool.k.upload(rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype]))
    pool.v.upload(rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype]))
    # first call: 12 rows up to 2000 keys over a 128-block table
    t1, r1 = batch(rng, [1, 15, 16, 17, 64, 65, 300, 700, 1000, 1500, 2000, 33], n_blocks, 128)
    q1 = (2.0 * rng.standard_normal((len(r1), nq, d))).astype(NP[dtype])
    want, got = both(ctx, pool, q1, t1, r1, nq, 1.0 / np.sqrt(d))
    assert not np.isnan(want).any()
    assert_bits_equal(got, want, what=f"first call {dtype} {nq}/{nk}x{d}")
    # second call: fewer rows, shorter ranges, a narrower table
    t2, r2 = batch(rng, [5, 129, 40], n_blocks, 20)
    q2 = (2.0 * rng.standard_normal((len(r2), nq, d))).astype(NP[dtype])
    want2, got2 = both(ctx, pool, q2, t2, r2, nq, 0.125)
    assert_bits_equal(got2, want2, what=f"second call {dtype} {nq}/{nk}x{d}")


def test_noalloc_decode_step_shape_and_a_row_alone(ctx):
    """Config B's decode batch (32 rows of 32/8 x 128 f32 at 4096 keys), then
    one row of it alone: the row's bits are the same in both."""
    rng = np.random.default_rng(11)
    nq, nk, d, n_blocks = 32, 8, 128, 1024
    pool = ops.KvPool(ctx, n_blocks, nk, d, np.float32)
    pool.k.upload(rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32))
    pool.v.upload(rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32))
    tables = np.stack([rng.choice(n_blocks, 256, replace=False) for _ in range(32)]).astype(np.uint32)
    ranges = np.tile(np.array([[0, 4096]], np.int32), (32, 1))
    q = rng.standard_normal((32, nq, d)).astype(np.float32)
    want, got = both(ctx, pool, q, tables, ranges, nq, 1.0 / np.sqrt(d))
    assert_bits_equal(got, want, what="batch 32")
    want1, got1 = both(ctx, pool, q[7:8], tables[7:8], ranges[7:8], nq, 1.0 / np.sqrt(d))
    assert_bits_equal(got1, want1, what="row alone")
    assert_bits_equal(got1[0], got[7], what="row alone vs in the batch")


def test_noalloc_refuses_a_call_beyond_the_scratch(ctx):
    """64 rows x 32 heads at 65536 f32 keys would need about 545 MB of
    partials: refused on the host, before any launch."""
    nq, nk, d, n_blocks, width = 32, 8, 128, 64, 4096
    rows = 64
    pool = ops.KvPool(ctx, n_blocks, nk, d, np.float32)
    tables = ctx.array(np.zeros((rows, width), np.uint32))
    ranges = ctx.array(np.tile(np.array([[0, 16]], np.int32), (rows, 1)))
    q = ctx.array(np.zeros((rows, nq, d), np.float32))
    with pytest.raises(hip.CucaError) as e:
        pool.decode_noalloc(q, tables, ranges, nq, 0.1)
    assert e.value.status == hip.INVALID_ARG
    assert "scratch" in e.value.message and str(hip.NOALLOC_SCRATCH_BYTES) in e.value.message
    ctx.check_device()
