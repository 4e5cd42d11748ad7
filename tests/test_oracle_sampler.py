"""Pinning the oracle's end of a step (cap_logits, greedy, select_top_k,
sample) and checking the library's host-side sampler finish against it.

Pins, from the reference's own tests (sampler.rs:364-651):
- SplitMix64's published vector for seed 0 (0xE220A8397B1DCDAF,
  0x6E789E6AA1B965F4) and next_f32 in [0, 1);
- greedy: the first maximum wins ([1, 3, 3, 2] -> 1), temperature <= 0 is
  the argmax, a NaN never wins, an all -inf row gives 0;
- top-k 1 is the argmax for every seed, a tiny top-p is the argmax, top-k 3
  draws only the three best, the same seed repeats a sequence and another
  seed does not, masked (-inf) logits are never drawn, an underflowing
  softmax keeps the maximum;
- select_top_k equals the k best of a full sort among many equal logits
  (ties by ascending id), for k = 1, 2, 7, 40, 333, 999;
- cap_logits: candle's affine multiplies by f32(1 / scale) (a division
  differs for some values: a planted mistake the test rejects), the
  soft-cap keeps |v| below the cap and is the identity to first order.
The library's cuca_hip_sample_candidates (host code, no GPU) is then held to
the oracle's sample, bit for bit in the drawn ids, over seeds, temperatures,
top-k and top-p values, with its candidates from the oracle's select_top_k.
"""
import ctypes

import numpy as np
import pytest

from cuca_amd import hip
from oracle import oracle as O


def ref_logits():
    return np.array([0.1, 2.0, 0.5, 1.9, -1.0, 1.95, 0.0], np.float32)


def test_splitmix64_matches_the_published_vector():
    r = O.SplitMix64(0)
    assert r.next_u64() == 0xE220A8397B1DCDAF
    assert r.next_u64() == 0x6E789E6AA1B965F4
    r = O.SplitMix64(42)
    vals = [r.next_f32() for _ in range(1000)]
    assert all(0.0 <= v < 1.0 for v in vals)


def test_greedy_known_answers():
    assert O.greedy([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.greedy(ref_logits()) == 1
    assert O.greedy([np.nan, 1.0, np.nan]) == 1
    assert O.greedy([np.nan, np.nan]) == 0
    assert O.greedy([-np.inf] * 5) == 0
    assert O.greedy([-np.inf, np.inf, np.inf]) == 1
    assert O.greedy([0.0, -0.0, 0.0]) == 0


def test_sample_known_answers():
    assert O.sample(ref_logits(), 0.0, 0, 1.0, O.SplitMix64(1)) == 1
    assert O.sample([1.0, 3.0, 3.0, 2.0], 0.0, 0, 1.0, O.SplitMix64(1)) == 1
    for seed in range(64):
        assert O.sample(ref_logits(), 1.5, 1, 1.0, O.SplitMix64(seed)) == 1
        assert O.sample(ref_logits(), 1.0, 0, 1e-6, O.SplitMix64(seed)) == 1
    rng = O.SplitMix64(3)
    assert all(O.sample(ref_logits(), 5.0, 3, 1.0, rng) in (1, 3, 5) for _ in range(200))

    def run(seed):
        rng = O.SplitMix64(seed)
        return [O.sample(ref_logits(), 1.0, 5, 0.95, rng) for _ in range(32)]
    assert run(7) == run(7) and run(7) != run(8)


def test_masked_logits_are_never_drawn():
    base = np.full(64, -np.inf, np.float32)
    base[[3, 17, 29, 44]] = [2.0, 1.5, 1.0, 0.5]
    rng = O.SplitMix64(101)
    for top_k in (0, 2, 16, 50):
        for top_p in (0.5, 0.99, 1.0):
            for _ in range(32):
                assert O.sample(base, 0.8, top_k, top_p, rng) in (3, 17, 29, 44)
    under = np.full(8, -np.inf, np.float32)
    under[2], under[5] = 1000.0, -1000.0
    assert O.sample(under, 1.0, 5, 1.0, rng) == 2
    assert O.sample(np.full(8, -np.inf, np.float32), 1.0, 0, 1.0, rng) == 0


def test_select_top_k_is_the_full_sort():
    rng = O.SplitMix64(23)
    logits = np.floor(np.array([rng.next_f32() * 16.0 for _ in range(1000)], np.float32))
    order = sorted(range(1000), key=lambda i: (-float(logits[i]), i))
    for k in (1, 2, 7, 40, 333, 999):
        vals, ids = O.select_top_k(logits, 1.0, k)
        assert ids.tolist() == order[:k]
        assert np.array_equal(vals, logits[ids])
    # temperature scales first (an IEEE division), non-finite values are skipped
    x = np.array([1.0, np.inf, -np.inf, np.nan, 3.0, -0.0, 0.0], np.float32)
    vals, ids = O.select_top_k(x, 0.7, 10)
    assert ids.tolist() == [4, 0, 6, 5]
    assert np.array_equal(vals, (x[ids] / np.float32(0.7)).astype(np.float32))


def test_cap_logits():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(100000) * 40).astype(np.float32)
    got = O.cap_logits(v, logit_scale=3.0)
    want = (v * np.float32(1.0 / 3.0)).astype(np.float32)
    assert np.array_equal(got, want)
    assert not np.array_equal(got, (v / np.float32(3.0)).astype(np.float32))  # the planted mistake
    assert np.array_equal(O.cap_logits(v, logit_mult=0.5), (v * np.float32(0.5)).astype(np.float32))
    c = O.cap_logits(v, softcap=30.0)
    assert np.all(np.abs(c) < 30.0 + 1e-3)
    small = np.array([1e-3, -2e-3], np.float32)
    assert np.allclose(O.cap_logits(small, softcap=30.0), small, rtol=1e-6)
    assert np.array_equal(O.cap_logits(np.array([-0.0], np.float32), logit_scale=2.0).view(np.uint32),
                          np.zeros(1, np.uint32))  # + 0 turns -0 into +0, as candle's affine


@pytest.mark.parametrize("temperature,top_k,top_p", [(1.0, 40, 0.95), (0.7, 5, 1.0), (1.3, 1, 0.9),
                                                     (0.8, 100, 0.5), (2.0, 7, 1e-6)])
def test_the_library_host_finish_is_the_reference_sample(temperature, top_k, top_p):
    """select_top_k (oracle) + cuca_hip_sample_candidates == sample, drawn
    id for drawn id, over 200 draws of one generator."""
    rng = np.random.default_rng(top_k)
    logits = (rng.standard_normal(5000) * 3).astype(np.float32)
    logits[rng.integers(0, 5000, 50)] = -np.inf
    a, b = O.SplitMix64(99), ctypes.c_uint64(99)
    vals, ids = O.select_top_k(logits, temperature, top_k)
    fallback = O.greedy(logits)
    for _ in range(200):
        want = O.sample(logits, temperature, top_k, top_p, a)
        got = hip.sample_candidates(vals, ids, top_p, fallback, b)
        assert got == want
    assert b.value == a.state.value


def test_the_library_host_finish_without_candidates_draws_the_fallback():
    st = ctypes.c_uint64(5)
    assert hip.sample_candidates(np.zeros(0, np.float32), np.zeros(0, np.uint32), 0.9, 7, st) == 7
    ref = O.SplitMix64(5)
    ref.next_u64()
    assert st.value == ref.state.value  # the draw still advances the generator
