"""Paged decode attention on the GPU against the oracle (attend_paged_rows
restated, per row).

Bar: |got - want| <= 1e-5 |want| + 1e-5 max|v| (f32), 2 f16 ulps + the same
floor (f16), where max|v| is the largest value magnitude of the row's range
in that KV head: the output is a convex combination of the values, and the
two sides sum the scores and the softmax in different orders (the reference
holds its own GPU kernel to 1e-4 absolute, gpu.rs:8289-8350).

Covers the reference GPU test's cases (scrambled blocks [7, 2, 11, 0, 9,
4], lengths around block boundaries, a window floor with released blocks
before it, heads 4/2 d 16, 6/2 d 8, 2/2 d 32 -- the generic kernel), the
configs' head layouts (GQA groups 2, 4, 8; head_dim 128 and 256; f32 and
f16) over contexts of 1 to 1000 keys, a row's bits alone and in a batch,
bad ranges and blocks, workspace checks and config C at 8192 keys.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.float16}


def floor_of(tables, ranges, pool_v, n_head):
    """1e-5 x max |v| over each row's range, per (row, head), broadcast to d."""
    rows = len(ranges)
    n_kv, d = pool_v.shape[1], pool_v.shape[3]
    f = np.zeros((rows, n_head, d))
    for r in range(rows):
        lo, hi = ranges[r]
        vals = O.gather(tables[r], lo, hi, pool_v).astype(np.float64)  # [n_kv, l, d]
        vmax = np.abs(vals).max(axis=(1, 2))
        f[r] = 1e-5 * np.repeat(vmax, n_head // n_kv)[:, None]
    return f


def run(ctx, q, pk, pv, tables, ranges, n_head, scale):
    rows, _, d = q.shape
    n_blocks, n_kv = pk.shape[0], pk.shape[1]
    pool = ops.KvPool(ctx, n_blocks, n_kv, d, q.dtype)
    pool.k.upload(pk)
    pool.v.upload(pv)
    out = pool.decode(ctx.array(q), ctx.array(tables.astype(np.uint32)),
                      ctx.array(ranges.astype(np.int32)), n_head, scale)
    ctx.check_device()
    return out.numpy()


def check(ctx, q, pk, pv, tables, ranges, n_head, scale):
    got = run(ctx, q, pk, pv, tables, ranges, n_head, scale)
    want = O.paged_attention(q, tables, ranges, pk, pv, scale, threads=8)
    assert_close(got, want, floor=floor_of(tables, ranges, pv, n_head), what="attention")
    return got


def test_the_reference_gpu_test_cases(ctx):
    rng = np.random.default_rng(7)
    n_blocks = 12
    scrambled = [7, 2, 11, 0, 9, 4]
    for nh, nkv, d in [(4, 2, 16), (6, 2, 8), (2, 2, 32)]:
        pk = rng.standard_normal((n_blocks, nkv, 16, d)).astype(np.float32)
        pv = rng.standard_normal((n_blocks, nkv, 16, d)).astype(np.float32)
        tables, ranges = [], []
        for hi in [1, 2, 15, 16, 17, 31, 32, 33, 70]:
            los = sorted({0, max(hi - 5, 0)} | ({16} if hi > 17 else set()))
            for lo in los:
                t = list(scrambled)
                t[:lo // 16] = [O.NO_BLOCK] * (lo // 16)
                tables.append(t)
                ranges.append((lo, hi))
        tables, ranges = np.array(tables, np.uint32), np.array(ranges, np.int32)
        q = (4.0 * rng.standard_normal((len(ranges), nh, d))).astype(np.float32)
        check(ctx, q, pk, pv, tables, ranges, nh, 1.0 / np.sqrt(d))


def make_batch(rng, lengths, n_blocks, width):
    """Rows with the given key counts, some with a window floor, over
    scrambled blocks of a shared pool."""
    tables = np.full((len(lengths), width), O.NO_BLOCK, np.uint32)
    ranges = np.zeros((len(lengths), 2), np.int32)
    for r, hi in enumerate(lengths):
        nb = (hi + 15) // 16
        tables[r, :nb] = rng.choice(n_blocks, nb, replace=False)
        lo = 0 if r % 3 else max(0, hi - 100)   # every third row: a window of 100
        tables[r, :lo // 16] = O.NO_BLOCK
        ranges[r] = (lo, hi)
    return tables, ranges


@pytest.mark.parametrize("cfg_name,dtype", [("A", "f32"), ("B", "f32"), ("C", "f16"),
                                            ("D", "f32"), ("D", "f16"), ("E", "f32"),
                                            ("E", "f16")])
def test_configs(ctx, cfg_name, dtype):
    cfg = W.CONFIGS[cfg_name]
    rng = np.random.default_rng(cfg["seed"])
    nq, nk, d = cfg["nq"], cfg["nk"], cfg["head_dim"]
    lengths = [1, 15, 16, 17, 63, 64, 65, 129, 300, 1000]
    n_blocks = 256
    tables, ranges = make_batch(rng, lengths, n_blocks, 64)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = (2.0 * rng.standard_normal((len(lengths), nq, d))).astype(NP[dtype])
    check(ctx, q, pk, pv, tables, ranges, nq, 1.0 / np.sqrt(d))


def test_a_row_is_bit_identical_alone_and_in_a_batch(ctx):
    rng = np.random.default_rng(8)
    nq, nk, d, n_blocks = 32, 8, 128, 128
    tables, ranges = make_batch(rng, [700, 5, 64, 333], n_blocks, 48)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    q = rng.standard_normal((4, nq, d)).astype(np.float32)
    all_rows = run(ctx, q, pk, pv, tables, ranges, nq, 0.1)
    for r in range(4):
        # alone, and with a narrower table (the chunking follows the range only)
        one = run(ctx, q[r:r + 1], pk, pv, tables[r:r + 1, :44], ranges[r:r + 1], nq, 0.1)
        assert_bits_equal(one[0], all_rows[r], f"row {r}")


@pytest.mark.parametrize("dtype,width", [("f32", 8), ("f16", 16)])
def test_one_part_rows_skip_the_merge(ctx, dtype, width):
    """A call whose rows all fit one part (a table of at most one part's
    blocks: 128 f32 / 256 f16 keys at 32/8 heads of 128) has the split write
    the outputs: one launch, the bits of the merge path (the same rows next
    to a long row), within the oracle's bar; a bad range gives the merge
    path's zero row."""
    rng = np.random.default_rng(width)
    nq, nk, d, n_blocks = 32, 8, 128, 96
    lengths = [1, 5, 16, 17, 100, width * 16]
    tables, ranges = make_batch(rng, lengths, n_blocks, width)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = (2.0 * rng.standard_normal((len(lengths), nq, d))).astype(NP[dtype])
    ctx.sync()
    ctx.profile_start(8)
    got = check(ctx, q, pk, pv, tables, ranges, nq, 1.0 / np.sqrt(d))
    names = [k for k, _ in ctx.profile_stop()]
    assert len(names) == 1 and names[0].startswith("cuca_attn_split"), names
    # the same rows in a call with a long row take the merge
    lt, lr = make_batch(rng, [700], n_blocks, 48)
    wide = np.full((len(lengths) + 1, 48), O.NO_BLOCK, np.uint32)
    wide[:len(lengths), :width] = tables
    wide[len(lengths)] = lt[0]
    ql = (2.0 * rng.standard_normal((1, nq, d))).astype(NP[dtype])
    merged = run(ctx, np.concatenate([q, ql]), pk, pv, wide, np.concatenate([ranges, lr]), nq, 1.0 / np.sqrt(d))
    assert_bits_equal(got, merged[:len(lengths)], "one-part rows vs the merge path")
    # a bad range: zeros, as the merge writes them, and reported
    bad = ranges.copy()
    bad[2] = (9, 9)
    for tb, rg, qq in ((tables, bad, q), (wide, np.concatenate([bad, lr]), np.concatenate([q, ql]))):
        with pytest.raises(hip.CucaError, match="empty key range"):
            run(ctx, qq, pk, pv, tb, rg, nq, 0.1)
        pool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
        pool.k.upload(pk)
        pool.v.upload(pv)
        out = pool.decode(ctx.array(qq), ctx.array(tb.astype(np.uint32)), ctx.array(rg.astype(np.int32)), nq, 0.1)
        with pytest.raises(hip.CucaError):
            ctx.check_device()
        assert not np.any(out.numpy()[2]), "bad row not zero"


def test_bad_blocks_and_ranges_are_reported(ctx):
    rng = np.random.default_rng(9)
    pk = rng.standard_normal((4, 1, 16, 64)).astype(np.float32)
    q = rng.standard_normal((2, 2, 64)).astype(np.float32)
    tables = np.array([[0, 1], [2, 9]], np.uint32)     # block 9 is outside a pool of 4
    with pytest.raises(hip.CucaError, match="attention row 1: position 16 has no K/V block"):
        run(ctx, q, pk, pk, tables, np.array([[0, 20], [0, 20]], np.int32), 2, 0.1)
    with pytest.raises(hip.CucaError, match="attention row 0: empty key range"):
        run(ctx, q, pk, pk, tables, np.array([[5, 5], [0, 3]], np.int32), 2, 0.1)
    with pytest.raises(hip.CucaError, match="attention row 1: empty key range, or one past"):
        run(ctx, q, pk, pk, tables, np.array([[0, 3], [0, 33]], np.int32), 2, 0.1)


def test_host_checks(ctx):
    pool = ops.KvPool(ctx, 4, 2, 64, np.float32)
    q = ctx.array(np.zeros((1, 4, 64), np.float32))
    tab = ctx.array(np.zeros((1, 2), np.uint32))
    rng = ctx.array(np.array([[0, 5]], np.int32))
    need = hip.paged_decode_workspace(1, 4, 64, 2)
    assert need == 1 * 4 * 1 * 66 * 4
    small = ctx.empty((need - 4,), np.uint8)
    with pytest.raises(hip.CucaError, match="workspace of"):
        pool.decode(q, tab, rng, 4, 0.1, workspace=small)
    with pytest.raises(hip.CucaError, match="query shape mismatch"):
        ctx.paged_decode(q.ptr, pool.k.ptr, pool.v.ptr, 4, tab.ptr, 2, rng.ptr, 1, 3, 2, 64, 0.1,
                         small.ptr, need, q.ptr, hip.F32)


def test_config_c_at_8192_keys(ctx):
    cfg = W.CONFIGS["C"]
    rng = np.random.default_rng(10)
    nq, nk, d = cfg["nq"], cfg["nk"], cfg["head_dim"]
    rows, ctx_len = 4, 8192
    n_blocks = rows * ctx_len // 16 + 16
    tables = rng.permutation(n_blocks)[:rows * ctx_len // 16].reshape(rows, -1).astype(np.uint32)
    ranges = np.array([[0, ctx_len], [0, ctx_len - 1], [4096, ctx_len], [0, 5000]], np.int32)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float16)
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float16)
    q = rng.standard_normal((rows, nq, d)).astype(np.float16)
    check(ctx, q, pk, pv, tables, ranges, nq, 1.0 / np.sqrt(d))


def decode_raw(ctx, q_dev, q_ld, pool, tables, ranges, n_head, scale, out, ws, ws_bytes, dtype):
    ctx.paged_decode(q_dev.ptr, pool.k.ptr, pool.v.ptr, pool.n_blocks, tables.ptr, tables.shape[1],
                     ranges.ptr, ranges.shape[0], n_head, pool.n_kv_head, pool.head_dim, scale,
                     ws.ptr, ws_bytes, out.ptr, dtype, q_ld=q_ld)


def test_query_rows_read_in_place_from_a_fused_qkv_row(ctx):
    """q at the start of wider rows (a fused Q|K|V projection's output, row
    stride q_ld): the same bits as the packed rows."""
    rng = np.random.default_rng(11)
    nq, nk, d, n_blocks = 32, 8, 128, 64
    for dtype in ("f32", "f16"):
        tables, ranges = make_batch(rng, [300, 17, 64], n_blocks, 24)
        pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
        pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
        q = rng.standard_normal((3, nq, d)).astype(NP[dtype])
        packed = run(ctx, q, pk, pv, tables, ranges, nq, 0.09)
        q_ld = (nq + 2 * nk) * d
        wide = rng.standard_normal((3, q_ld)).astype(NP[dtype])
        wide[:, :nq * d] = q.reshape(3, -1)
        pool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
        pool.k.upload(pk)
        pool.v.upload(pv)
        need = hip.paged_decode_workspace(3, nq, d, tables.shape[1])
        ws, out = ctx.empty((need,), np.uint8), ctx.empty((3, nq, d), NP[dtype])
        decode_raw(ctx, ctx.array(wide), q_ld, pool, ctx.array(tables), ctx.array(ranges), nq, 0.09,
                   out, ws, need, hip.dtype_code(NP[dtype]))
        ctx.check_device()
        assert_bits_equal(out.numpy(), packed, f"strided q {dtype}")
    with pytest.raises(hip.CucaError, match="q row stride"):
        decode_raw(ctx, ctx.array(wide), nq * d - 1, pool, ctx.array(tables), ctx.array(ranges), nq,
                   0.09, out, ws, need, hip.F16)


def test_many_rows_keep_each_rows_bits(ctx):
    """8200 rows x 8 KV heads (65600 (row, head) merges, ragged ranges of 1
    to 608 keys): the first rows carry the bits the same rows get in a call
    of 64 rows, and sampled rows meet the oracle bar."""
    rng = np.random.default_rng(12)
    nh, nk, d, n_blocks, width = 8, 8, 64, 48, 38
    rows = 8200
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    tables = np.stack([rng.choice(n_blocks, width, replace=False) for _ in range(rows)]).astype(np.uint32)
    hi = rng.integers(1, width * 16 + 1, rows)
    lo = np.where(np.arange(rows) % 4 == 0, np.maximum(hi - 300, 0), 0)
    ranges = np.stack([lo, hi], 1).astype(np.int32)
    q = rng.standard_normal((rows, nh, d)).astype(np.float32)
    big = run(ctx, q, pk, pv, tables, ranges, nh, 0.125)
    small = run(ctx, q[:64], pk, pv, tables[:64], ranges[:64], nh, 0.125)
    assert_bits_equal(small, big[:64], "64-row call vs 8200-row call")
    pick = np.array([0, 1, 2, 3, 4097, rows - 1])
    want = O.paged_attention(q[pick], tables[pick], ranges[pick], pk, pv, 0.125, threads=8)
    assert_close(big[pick], want, floor=floor_of(tables[pick], ranges[pick], pv, nh), what="attention")


def test_repeated_calls_and_graph_replays_keep_their_bits(ctx):
    """Calls in a row and replays of a captured call (split and merge
    launches; eager work and synchronizations between the replays) all give
    the first call's bits."""
    rng = np.random.default_rng(13)
    nq, nk, d, n_blocks = 32, 8, 128, 96
    tables, ranges = make_batch(rng, [1000, 1, 129, 64, 500], n_blocks, 64)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    q = rng.standard_normal((5, nq, d)).astype(np.float32)
    first = check(ctx, q, pk, pv, tables, ranges, nq, 0.1)
    pool = ops.KvPool(ctx, n_blocks, nk, d, np.float32)
    pool.k.upload(pk)
    pool.v.upload(pv)
    need = hip.paged_decode_workspace(5, nq, d, tables.shape[1])
    ws, out = ctx.empty((need,), np.uint8), ctx.empty((5, nq, d), np.float32)
    dq, dt, dr = ctx.array(q), ctx.array(tables), ctx.array(ranges)
    for i in range(3):
        decode_raw(ctx, dq, nq * d, pool, dt, dr, nq, 0.1, out, ws, need, hip.F32)
        ctx.check_device()
        assert_bits_equal(out.numpy(), first, f"call {i}")
    ctx.graph_begin()
    decode_raw(ctx, dq, nq * d, pool, dt, dr, nq, 0.1, out, ws, need, hip.F32)
    g = ctx.graph_end()
    try:
        for i in range(4):
            out.upload(np.zeros((5, nq, d), np.float32))
            g.launch()
            ctx.sync()
            assert_bits_equal(out.numpy(), first, f"replay {i}")
            decode_raw(ctx, dq, nq * d, pool, dt, dr, nq, 0.1, out, ws, need, hip.F32)  # eager between
            ctx.check_device()
    finally:
        g.destroy()


@pytest.mark.parametrize("dtype,nq,nk,d", [("f32", 6, 2, 40), ("f32", 32, 8, 128)])
def test_wide_tables_take_the_late_and_the_long_merge(ctx, dtype, nq, nk, d):
    """A block table wide enough that a row may have more than 256 parts
    (2200 blocks = 35200 keys: 550 parts of the generic kernel's 64
    positions, 275 of the f32 d128 kernel's 128), so the merge cannot issue
    its loads before the range is known (the late short path), and rows
    long enough for the long path (more than 256 parts: 20000 keys for the
    generic kernel, 34000 for d128).  The workspace starts filled with NaN,
    so parts past a row's count must be selected away, not multiplied by 0.
    A short row gives the same bits with a narrow table."""
    rng = np.random.default_rng(14 + d)
    n_blocks, width = 2200, 2200
    lengths = [300, 20000, 34000, 1, 4097]
    tables = np.full((len(lengths), width), O.NO_BLOCK, np.uint32)
    ranges = np.zeros((len(lengths), 2), np.int32)
    for r, hi in enumerate(lengths):
        nb = (hi + 15) // 16
        tables[r, :nb] = rng.choice(n_blocks, nb, replace=False)
        lo = hi - 1000 if r == 4 else 0   # one row with a window floor
        tables[r, :lo // 16] = O.NO_BLOCK
        ranges[r] = (lo, hi)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(NP[dtype])
    q = (2.0 * rng.standard_normal((len(lengths), nq, d))).astype(NP[dtype])
    pool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
    pool.k.upload(pk)
    pool.v.upload(pv)
    need = hip.paged_decode_workspace(len(lengths), nq, d, width)
    ws = ctx.array(np.full(need // 4, np.nan, np.float32))
    dt, dr = ctx.array(tables), ctx.array(ranges)
    got = pool.decode(ctx.array(q), dt, dr, nq, 1.0 / np.sqrt(d), workspace=ws).numpy()
    ctx.check_device()
    want = O.paged_attention(q, tables, ranges, pk, pv, 1.0 / np.sqrt(d), threads=8)
    assert_close(got, want, floor=floor_of(tables, ranges, pv, nq), what="wide-table attention")
    # the 300-key row with a 20-block table: the early short path, same bits
    narrow = run(ctx, q[:1], pk, pv, tables[:1, :20], ranges[:1], nq, 1.0 / np.sqrt(d))
    assert_bits_equal(narrow[0], got[0], "narrow vs wide table")
