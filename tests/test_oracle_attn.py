"""The oracle's paged attention (attend_paged_rows restated) pinned against
the mathematics and the reference's own test.

- paged_attention_matches_contiguous_attention (cpu/paged_attn.rs:413-480):
  attention over scrambled blocks equals attention over the same keys laid
  out contiguously, within 1e-5.  Restated with the contiguous side computed
  in f64 numpy (textbook softmax(q k^T * scale) v, with the grouped heads
  h -> h / (n_head / n_kv)), at the reference test's shapes, lengths and
  range floors.
- Exact special cases: one key -> its value, bit for bit (p = 1, acc / 1);
  equal scores (q = 0) -> the mean of the values.
- The f64 check has power: a planted mistake (the GQA map h % n_kv, or the
  scale left out) misses it by far more than the tolerance.
- Bad ranges (empty, NO_BLOCK, past the table) are rejected before anything
  is computed.
"""
import numpy as np
import pytest

from oracle import oracle as O


def contiguous_f64(q, keys, values, lo, hi, scale, gqa=None):
    """q [n_head, d]; keys/values [n_kv, l, d]; positions lo..hi."""
    n_head, d = q.shape
    n_kv = keys.shape[0]
    group = n_head // n_kv
    gqa = gqa or (lambda h: h // group)
    out = np.empty((n_head, d))
    for h in range(n_head):
        k = keys[gqa(h), lo:hi].astype(np.float64)
        v = values[gqa(h), lo:hi].astype(np.float64)
        s = k @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = p @ v / p.sum()
    return out


def scrambled(rng, n_head, n_kv, d, l, dtype=np.float32):
    blocks = -(-l // O.KV_BLOCK)
    table = np.array([(b * 5 + 3) % 11 for b in range(blocks)], np.uint32)
    pk = np.zeros((11, n_kv, O.KV_BLOCK, d), dtype)
    pv = np.zeros_like(pk)
    keys = rng.standard_normal((n_kv, l, d)).astype(dtype)
    values = rng.standard_normal((n_kv, l, d)).astype(dtype)
    O.store_rows(table, 0, keys, pk)
    O.store_rows(table, 0, values, pv)
    return table, pk, pv, keys, values


@pytest.mark.parametrize("n_head,n_kv,d", [(4, 2, 8), (8, 1, 16), (3, 3, 5)])
def test_matches_contiguous_attention_like_the_reference_test(n_head, n_kv, d):
    rng = np.random.default_rng(42)
    for l in [1, 2, 15, 16, 17, 33, 50]:
        table, pk, pv, keys, values = scrambled(rng, n_head, n_kv, d, l)
        for lo in sorted({0, l // 3, l // 2}):
            if lo >= l:
                continue
            q = (2.0 * rng.standard_normal((1, n_head, d))).astype(np.float32)
            scale = 1.0 / np.sqrt(d)
            got = O.paged_attention(q, table[None], np.array([[lo, l]]), pk, pv, scale)
            want = contiguous_f64(q[0], keys, values, lo, l, scale)
            assert np.max(np.abs(got[0] - want)) <= 1e-5, (n_head, n_kv, d, l, lo)


def test_one_key_gives_its_value_exactly_and_equal_scores_the_mean():
    rng = np.random.default_rng(1)
    table, pk, pv, keys, values = scrambled(rng, 4, 2, 16, 40)
    q = rng.standard_normal((1, 4, 16)).astype(np.float32)
    got = O.paged_attention(q, table[None], np.array([[17, 18]]), pk, pv, 0.25)
    for h in range(4):
        assert np.array_equal(got[0, h], values[h // 2, 17])
    got = O.paged_attention(np.zeros_like(q), table[None], np.array([[3, 40]]), pk, pv, 0.25)
    want = values[:, 3:40].astype(np.float64).mean(axis=1)
    assert np.max(np.abs(got[0] - np.repeat(want, 2, axis=0))) <= 2e-6


def test_the_check_rejects_planted_mistakes():
    rng = np.random.default_rng(2)
    table, pk, pv, keys, values = scrambled(rng, 8, 2, 16, 45)
    q = (2.0 * rng.standard_normal((1, 8, 16))).astype(np.float32)
    got = O.paged_attention(q, table[None], np.array([[0, 45]]), pk, pv, 0.25)[0]
    wrong_map = contiguous_f64(q[0], keys, values, 0, 45, 0.25, gqa=lambda h: h % 2)
    no_scale = contiguous_f64(q[0], keys, values, 0, 45, 1.0)
    assert np.max(np.abs(got - wrong_map)) > 1e-2
    assert np.max(np.abs(got - no_scale)) > 1e-2


def test_f16_pools_are_the_f32_computation_on_the_widened_values():
    rng = np.random.default_rng(3)
    table, pk, pv, keys, values = scrambled(rng, 4, 1, 32, 30, np.float16)
    q = rng.standard_normal((2, 4, 32)).astype(np.float16)
    got = O.paged_attention(q, np.stack([table, table]), np.array([[0, 30], [5, 29]]), pk, pv, 0.2)
    want = O.paged_attention(q.astype(np.float32), np.stack([table, table]),
                             np.array([[0, 30], [5, 29]]), pk.astype(np.float32),
                             pv.astype(np.float32), 0.2)
    assert np.array_equal(got, want.astype(np.float16))


@pytest.mark.parametrize("table,lo,hi", [
    ([3, 7], 5, 5),               # empty
    ([3, O.NO_BLOCK], 10, 20),    # a released block in the range
    ([3], 10, 20),                # past the table
])
def test_bad_ranges_are_rejected(table, lo, hi):
    pk = np.zeros((11, 1, 16, 8), np.float32)
    with pytest.raises(O.KvError):
        O.paged_attention(np.ones((1, 2, 8), np.float32), np.array([table], np.uint32),
                          np.array([[lo, hi]]), pk, pk, 1.0)
