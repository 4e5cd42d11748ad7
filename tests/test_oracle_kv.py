"""The oracle's paged K/V pool functions (store_rows, gather, store_kv)
pinned against the reference's own test and the layout's known answers.

- paged_attention_matches_contiguous_attention (cpu/paged_attn.rs:413-480)
  stores keys over scrambled block tables ((b * 5 + 3) % 11 in a pool of 11
  blocks) and requires the gathered range to equal the contiguous slice: the
  same shapes and lengths here, plus "the blocks the table does not name
  stay zero".
- A round trip cannot see a layout that store and gather both get wrong the
  same way (say rows and KV heads swapped), so the offsets are pinned by
  hand-computed known answers of row_offset (paged_attn.rs:33-38) for the
  [n_blocks][n_kv][16][d] pool; a planted transposed layout fails them.
- Missing blocks (NO_BLOCK, past the table, outside the pool) fail and
  write nothing (check_range, paged_attn.rs:42-65).
- store_kv's composition (cpu.rs:3028-3097): rotated Q, rotated K and V in
  the pools, V optionally normalised without a weight.
"""
import numpy as np
import pytest

from oracle import oracle as O


@pytest.mark.parametrize("n_kv,d", [(2, 8), (1, 16), (3, 5)])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_scrambled_tables_round_trip_like_the_reference_test(n_kv, d, dtype):
    rng = np.random.default_rng(42)
    for l in [1, 2, 15, 16, 17, 33, 50]:
        blocks = -(-l // O.KV_BLOCK)
        table = [(b * 5 + 3) % 11 for b in range(blocks)]
        pool = np.zeros((11, n_kv, O.KV_BLOCK, d), dtype)
        keys = rng.standard_normal((n_kv, l, d)).astype(dtype)
        O.store_rows(table, 0, keys, pool)
        for lo in [0, l // 3, l // 2]:
            assert np.array_equal(O.gather(table, lo, l, pool), keys[:, lo:])
        unused = sorted(set(range(11)) - set(table))
        assert not pool[unused].any()
        # the table's blocks hold exactly the stored rows (and zeros past l)
        assert np.count_nonzero(pool) == np.count_nonzero(keys)


def test_row_offset_known_answers():
    # pool of 5 blocks, 2 KV heads, d = 8; table [4, 2, 0]: position 21 is
    # row 5 of table[1] = block 2.  Element offsets, by hand:
    #   kvh 0: ((2*2 + 0)*16 + 5)*8 = 69*8 = 552
    #   kvh 1: ((2*2 + 1)*16 + 5)*8 = 85*8 = 680
    pool = np.zeros((5, 2, 16, 8), np.float32)
    src = np.arange(1, 17, dtype=np.float32).reshape(2, 1, 8)
    O.store_rows([4, 2, 0], 21, src, pool)
    flat = pool.reshape(-1)
    assert np.flatnonzero(flat).tolist() == list(range(552, 560)) + list(range(680, 688))
    assert flat[552:560].tolist() == list(range(1, 9))
    assert flat[680:688].tolist() == list(range(9, 17))
    # position 0 of table [4]: block 4, row 0: kvh 1 at ((4*2+1)*16)*8 = 1152
    pool[:] = 0
    O.store_rows([4], 0, src, pool)
    assert np.flatnonzero(flat).tolist() == list(range(1024, 1032)) + list(range(1152, 1160))


def _planted_transposed_store(table, start, src, pool):
    """A wrong layout, [n_blocks][16][n_kv][d]: round-trips with its own gather."""
    n_blocks, n_kv, bs, d = pool.shape
    view = pool.reshape(n_blocks, bs, n_kv, d)
    for r in range(src.shape[1]):
        p = start + r
        view[table[p // bs], p % bs] = src[:, r]


def test_a_planted_transposed_layout_fails_the_known_answers():
    pool = np.zeros((5, 2, 16, 8), np.float32)
    src = np.arange(1, 17, dtype=np.float32).reshape(2, 1, 8)
    _planted_transposed_store([4, 2, 0], 21, src, pool)
    got = np.flatnonzero(pool.reshape(-1)).tolist()
    assert got != list(range(552, 560)) + list(range(680, 688))


@pytest.mark.parametrize("table,start,rows", [
    ([3, O.NO_BLOCK], 0, 20),   # a released block
    ([3], 10, 10),              # past the table
    ([3, 11], 0, 20),           # outside the pool of 11
])
def test_missing_blocks_fail_and_write_nothing(table, start, rows):
    pool = np.zeros((11, 1, 16, 4), np.float32)
    with pytest.raises(O.KvError):
        O.store_rows(table, start, np.ones((1, rows, 4), np.float32), pool)
    assert not pool.any()
    with pytest.raises(O.KvError):
        O.gather(table, start, start + rows, pool)


def test_store_kv_composes_rope_norm_and_store():
    rng = np.random.default_rng(3)
    nq, nk, d = 4, 2, 16
    cos, sin = O.rope_tables(d, 1e4, 64)
    # two calls: rows 0..5 at cache 10.. (rope 10..), rows 5..12 at cache 0.. (rope 30..)
    calls = [(0, 10, 10, 5, [7, 1]), (5, 0, 30, 7, [2])]
    q = rng.standard_normal((12, nq, d)).astype(np.float32)
    k = rng.standard_normal((12, nk, d)).astype(np.float32)
    v = rng.standard_normal((12, nk, d)).astype(np.float32)
    pk = np.zeros((8, nk, 16, d), np.float32)
    pv = np.zeros_like(pk)
    qr = O.store_kv(q, k, v, cos, sin, O.ROPE_NEOX, d, calls, pk, pv, v_norm=True, eps=1e-6)
    pos = np.r_[np.arange(10, 15), np.arange(30, 37)].astype(np.int32)
    assert np.array_equal(qr, O.rope(q, cos, sin, pos, O.ROPE_NEOX))
    kr = O.rope(k, cos, sin, pos, O.ROPE_NEOX)
    assert np.array_equal(O.gather([7, 1], 10, 15, pk), kr[:5].transpose(1, 0, 2))
    assert np.array_equal(O.gather([2], 0, 7, pk), kr[5:].transpose(1, 0, 2))
    # V: x / sqrt(mean(x^2) + eps) in f64, to f32 rounding
    v64 = v.astype(np.float64)
    vn = v64 / np.sqrt((v64 ** 2).mean(-1, keepdims=True) + 1e-6)
    got = np.concatenate([O.gather([7, 1], 10, 15, pv), O.gather([2], 0, 7, pv)], axis=1)
    np.testing.assert_allclose(got, vn.transpose(1, 0, 2), rtol=2e-6, atol=1e-7)
    # the untouched blocks stay zero
    assert not pk[[0, 3, 4, 5, 6]].any() and not pv[[0, 3, 4, 5, 6]].any()
