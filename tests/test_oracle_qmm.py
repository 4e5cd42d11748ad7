"""Pinning the oracle's quantized matmul (QmmWeight, qmm.rs) for Q4_0 / Q8_0.

The reference holds no output vectors for its quantized matmul; its tests
(qmm/tests.rs) check the kernel against a scalar restatement of the module's
definition, an f64 product, and bounds.  The oracle is pinned here by:
- known answers for the activation quantisation (Acts::new, qmm.rs:1217-1343):
  a zero block, ties rounded away from zero (0.5 -> 1, 2.5 -> 3, not to
  even), the scale rounded to f16, a NaN ignored by the maximum and quantised
  to 0;
- hand-built weights and activations where the summation order of the
  definition (sixteen lanes, each sequential over the blocks, then the hsum
  tree h[i] = a[i] + a[i+8], ((h0+h4)+(h1+h5))+((h2+h6)+(h3+h7))) gives an
  answer that a per-block sum, a sequential lane sum, an adjacent-pairs tree
  or a fused multiply-add would not;
- the f64 product of the dequantised weights with the rounded activations
  (qmm/tests.rs:477-556) to 1e-4 of the output scale, with planted mistakes
  (the pair (l, l+1) instead of (l, l+16), swapped nibbles, no -8 offset, a
  transposed weight) that must miss it;
- the bound of qmm/tests.rs:558-592: against the exact product of the
  dequantised weights and the unrounded activations the error is at most
  0.6 * amax / 127 * sum |w| per block;
- row exactness: a row alone equals the row in any batch, a prefix of the
  weight rows equals the start of the product, zero activations give exact
  zeros (qmm/tests.rs:624-796).
"""
import numpy as np
import pytest

from cuca_amd import workloads as W
from oracle import oracle as O

F16 = np.float16


def f16_bytes(v):
    return np.array([v], np.float16).view(np.uint8)


def q8_block(d, quants):
    """A Q8_0 block: f16 scale d, 32 signed quants."""
    b = np.zeros(34, np.uint8)
    b[:2] = f16_bytes(d)
    b[2:] = np.asarray(quants, np.int8).view(np.uint8)
    return b


def dequant(w, qtype, n, k):
    return np.stack([O.dequant_row(qtype, w[r * O.row_bytes(qtype, k):(r + 1) * O.row_bytes(qtype, k)],
                                   1.0, k) for r in range(n)])


def rounded_acts(x):
    q, s = O.q8_acts(x)
    m, k = x.shape
    return q.astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)


def reference64(w, qtype, n, k, x):
    """qmm/tests.rs:424-439: dequantised weights times rounded activations, f64."""
    return rounded_acts(x) @ dequant(w, qtype, n, k).astype(np.float64).T


def noise(rng, m, k, scale):
    return (rng.uniform(-1.0, 1.0, (m, k)) * scale).astype(np.float32)


def awkward_acts(rng, m, k):
    """qmm/tests.rs:199-208: a zero block, an outlier, ties, a doubled max."""
    x = noise(rng, m, k, 3.0)
    x[:, :32] = 0.0
    x[:, 32 + 3] = 127.0
    x[:, 32 + 4] = 0.5
    x[:, 32 + 5] = -1.5
    if k >= 96:
        x[:, 64 + 10] = -9.0
        x[:, 64 + 20] = 9.0
    return x


# ---------------------------------------------------------------------------
# activation quantisation: known answers
# ---------------------------------------------------------------------------

def test_activation_quantisation_known_answers():
    x = np.zeros((1, 128), np.float32)
    # block 1: amax 127 -> d = 1 exactly; ties go away from zero
    x[0, 32 + 0] = 127.0
    x[0, 32 + 1] = 0.5
    x[0, 32 + 2] = -0.5
    x[0, 32 + 3] = 2.5
    x[0, 32 + 4] = -1.5
    x[0, 32 + 5] = 0.49999997
    # block 2: amax 9 twice (first negative): d = f32(9/127), quants +-127
    x[0, 64 + 10] = -9.0
    x[0, 64 + 20] = 9.0
    x[0, 64 + 21] = 4.5
    # block 3: a NaN is ignored by the maximum and quantises to 0
    x[0, 96 + 0] = np.nan
    x[0, 96 + 1] = 63.5
    x[0, 96 + 2] = -63.5
    q, s = O.q8_acts(x)
    assert s[0, 0] == 0.0 and not q[0, :32].any()
    assert s[0, 1] == 1.0
    assert q[0, 32:38].tolist() == [127, 1, -1, 3, -2, 0]
    d9 = np.float32(9.0) / np.float32(127.0)
    assert s[0, 2] == np.float32(F16(d9))
    assert q[0, 64 + 10] == -127 and q[0, 64 + 20] == 127
    # 4.5 * (1 / d9) = 63.5000...: f32 rounding decides, computed the same way
    id9 = np.float32(1.0) / d9
    t = np.float32(np.float32(4.5) * id9)
    want = int(np.trunc(t) + np.sign(t) * (abs(t - np.trunc(t)) >= 0.5))
    assert q[0, 64 + 21] == want
    assert s[0, 3] == np.float32(F16(np.float32(63.5) / np.float32(127.0)))
    assert q[0, 96:99].tolist() == [0, 127, -127]


def test_activation_scale_is_rounded_to_f16_and_saturates():
    # amax = 127 * (1 + 2^-12): d is not an f16 value, the stored scale is
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = np.float32(127.0 * (1.0 + 2.0 ** -12))
    q, s = O.q8_acts(x)
    assert s[0, 0] == np.float32(F16(np.float32(x[0, 0]) / np.float32(127.0)))
    assert s[0, 0] != x[0, 0] / np.float32(127.0)
    assert q[0, 0] == 127
    # an infinite element: d = inf, id = 0, every quant is 0 (inf * 0 = NaN -> 0)
    x = np.ones((1, 32), np.float32)
    x[0, 7] = np.inf
    q, s = O.q8_acts(x)
    assert np.isinf(s[0, 0]) and not q.any()


# ---------------------------------------------------------------------------
# the summation order, by hand
# ---------------------------------------------------------------------------

def _ones_block_x(d, entries):
    """32 activations whose block scale is exactly d (the amax element 127 * d
    sits at element 31, paired with a zero weight) and whose quants at the
    given elements are the given integers."""
    x = np.zeros(32, np.float32)
    x[31] = 127.0 * d
    for e, qv in entries.items():
        x[e] = qv * d
    return x


def test_lanes_are_sequential_over_blocks_then_the_tree():
    """Lane 0 gets +2^33 (block 0) and -2^33 (block 2); lane 8 gets 1
    (block 1).  The definition: lane 0 = (2^33 + 0) - 2^33 = 0, lane 8 = 1,
    hsum = 1.  A per-block total accumulated over blocks gives
    (2^33 + 1) - 2^33 = 0 (2^33 + 1 rounds to 2^33)."""
    k = 96
    x = np.concatenate([_ones_block_x(1024.0, {0: 64, 16: 64}),
                        _ones_block_x(1.0, {8: 1}),
                        _ones_block_x(1024.0, {0: 64, 16: 64})]).reshape(1, k)
    w0 = np.zeros(32, np.int8); w0[0] = 64; w0[16] = 64
    w1 = np.zeros(32, np.int8); w1[8] = 1
    w2 = np.zeros(32, np.int8); w2[0] = -64; w2[16] = -64
    w = np.concatenate([q8_block(1024.0, w0), q8_block(1.0, w1), q8_block(1024.0, w2)])
    got = O.qmm(w, O.Q8_0, 1, k, x)
    assert got[0, 0] == 1.0
    # the plausible alternatives give 0
    blocks = [np.float32(2.0 ** 33), np.float32(1.0), np.float32(-2.0 ** 33)]
    acc = np.float32(0.0)
    for b in blocks:
        acc = np.float32(acc + b)
    assert acc == 0.0


def test_the_lane_reduction_is_the_hsum_tree():
    """Lane 0 = 2^33, lane 8 = -2^33 (block 0, scale 2^20), lane 1 = 1
    (block 1, scale 1).  The tree adds a[0] + a[8] first: 0 + 1 = 1.  A
    sequential lane sum or an adjacent-pairs tree adds 2^33 + 1 first and
    ends at 0."""
    k = 64
    x = np.concatenate([_ones_block_x(1024.0, {0: 64, 16: 64, 8: 64, 24: 64}),
                        _ones_block_x(1.0, {1: 1})]).reshape(1, k)
    w0 = np.zeros(32, np.int8); w0[0] = 64; w0[16] = 64; w0[8] = -64; w0[24] = -64
    w1 = np.zeros(32, np.int8); w1[1] = 1
    w = np.concatenate([q8_block(1024.0, w0), q8_block(1.0, w1)])
    assert O.qmm(w, O.Q8_0, 1, k, x)[0, 0] == 1.0
    lanes = np.zeros(16, np.float32)
    lanes[0], lanes[8], lanes[1] = 2.0 ** 33, -2.0 ** 33, 1.0
    seq = np.float32(0.0)
    for v in lanes:
        seq = np.float32(seq + v)
    assert seq == 0.0
    pairs = lanes.copy()
    while pairs.size > 1:
        pairs = (pairs[0::2] + pairs[1::2]).astype(np.float32)
    assert pairs[0] == 0.0


def test_the_product_and_the_sum_are_rounded_separately():
    """acc = a + round(p * s), not round(a + p * s): with s = (2047/1024)^2
    (22 significant bits) and p = 16132 the product needs 36 bits.  The
    oracle must equal the separately rounded value and, for these inputs,
    differ from the fused one."""
    k = 64
    dsc = 2047.0 / 1024.0
    # block 0 puts a = round(127 * 127 * s) into lane 0; block 1 adds p * s
    x = np.concatenate([_ones_block_x(dsc, {0: 127}),
                        _ones_block_x(dsc, {0: 127, 16: 3})]).reshape(1, k)
    w0 = np.zeros(32, np.int8); w0[0] = 127
    w1 = np.zeros(32, np.int8); w1[0] = 127; w1[16] = 1
    w = np.concatenate([q8_block(dsc, w0), q8_block(dsc, w1)])
    q, sc = O.q8_acts(x)
    assert sc[0].tolist() == [np.float32(dsc)] * 2
    s = np.float32(np.float32(F16(dsc)) * sc[0, 0])
    a = np.float32(np.float32(127 * 127) * s)
    p = 127 * 127 + 1 * 3
    separate = np.float32(a + np.float32(np.float32(p) * s))
    fused = np.float32(float(a) + float(p) * float(s))
    assert separate != fused
    assert O.qmm(w, O.Q8_0, 1, k, x)[0, 0] == separate


def test_q4_0_nibbles_pair_element_i_with_i_plus_16():
    """Byte i of a Q4_0 block holds element i (low nibble) and element i+16
    (high nibble), each minus 8 (qmm.rs:240-263)."""
    k = 32
    blk = np.zeros(18, np.uint8)
    blk[:2] = f16_bytes(1.0)
    blk[2:] = 0x88  # every element 0
    blk[2 + 3] = 0x8B  # element 3 = 11 - 8 = 3, element 19 = 8 - 8 = 0
    blk[2 + 5] = 0x28  # element 5 = 0, element 21 = 2 - 8 = -6
    x = _ones_block_x(1.0, {3: 10, 21: 7, 4: 100, 19: 50}).reshape(1, k)
    # lane 3: 3*10 + 0*50 = 30; lane 5: 0 + (-6)*7 = -42; element 31 has weight 0
    assert O.qmm(blk, O.Q4_0, 1, k, x)[0, 0] == np.float32(30 - 42)


# ---------------------------------------------------------------------------
# against f64, with planted mistakes
# ---------------------------------------------------------------------------

SHAPES = [(10, 512, 7), (3, 256, 1), (600, 256, 5), (64, 768, 17), (10, 64, 7), (3, 32, 1),
          (64, 96, 17)]


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("n,k,m", SHAPES)
def test_matches_the_f64_reference(qtype, n, k, m):
    rng = np.random.default_rng(n * 1000 + k + m)
    w = W.quant_table(rng, n, k, qtype, (0.004, 0.012))
    x = noise(rng, m, k, 1.0)
    got = O.qmm(w, W.GGML_ID[qtype], n, k, x, threads=4)
    want = reference64(w, W.GGML_ID[qtype], n, k, x)
    scale = np.max(np.abs(want))
    assert np.max(np.abs(got - want)) <= 1e-4 * scale


def test_planted_mistakes_miss_the_f64_reference():
    rng = np.random.default_rng(5)
    n, k, m = 16, 256, 3
    for qtype in ("q4_0", "q8_0"):
        gid = W.GGML_ID[qtype]
        w = W.quant_table(rng, n, k, qtype, (0.004, 0.012))
        x = noise(rng, m, k, 1.0)
        xr = rounded_acts(x)
        want = reference64(w, gid, n, k, x)
        tol = 1e-4 * np.max(np.abs(want))
        got = O.qmm(w, gid, n, k, x)
        assert np.max(np.abs(got - want)) <= tol
        wd = dequant(w, gid, n, k).astype(np.float64)
        # the pair (l, l+1) instead of (l, l+16): element order within a block
        perm = np.concatenate([np.arange(0, 32, 2), np.arange(1, 32, 2)])
        wrong = xr @ wd.reshape(n, -1, 32)[:, :, perm].reshape(n, k).T
        assert np.max(np.abs(wrong - want)) > 10 * tol
        # a transposed (reversed) block order
        wrong = xr @ wd.reshape(n, -1, 32)[:, ::-1, :].reshape(n, k).T
        assert np.max(np.abs(wrong - want)) > 10 * tol
        if qtype == "q4_0":
            blocks = w.reshape(n, -1, 18)
            d = blocks[:, :, :2].copy().view(np.float16).astype(np.float64)
            nib = blocks[:, :, 2:]
            lo, hi = (nib & 15).astype(np.float64), (nib >> 4).astype(np.float64)
            swapped = np.concatenate([hi, lo], axis=2) - 8.0
            wrong = xr @ (swapped * d).reshape(n, k).T
            assert np.max(np.abs(wrong - want)) > 10 * tol
            no_offset = np.concatenate([lo, hi], axis=2)
            wrong = xr @ (no_offset * d).reshape(n, k).T
            assert np.max(np.abs(wrong - want)) > 10 * tol


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_the_error_is_bounded_by_the_activation_rounding(qtype):
    """qmm/tests.rs:558-592."""
    rng = np.random.default_rng(23)
    for n, k, m in [(12, 512, 5), (20, 256, 3)]:
        gid = W.GGML_ID[qtype]
        w = W.quant_table(rng, n, k, qtype, (0.004, 0.012))
        x = noise(rng, m, k, 1.0)
        for j in range(m):
            x[j, 7] = 6.0 * (j + 1)
        got = O.qmm(w, gid, n, k, x).astype(np.float64)
        wd = dequant(w, gid, n, k).astype(np.float64)
        exact = x.astype(np.float64) @ wd.T
        amax = np.abs(x.reshape(m, -1, 32)).max(axis=2).astype(np.float64)   # [m, nb]
        absw = np.abs(wd.reshape(n, -1, 32)).sum(axis=2)                      # [n, nb]
        bound = 0.6 * amax / 127.0 @ absw.T
        assert np.all(np.abs(got - exact) <= bound + 1e-5 * np.maximum(np.abs(exact), 1.0))


# ---------------------------------------------------------------------------
# row exactness, prefixes, zeros, errors
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_a_row_is_bit_identical_alone_and_in_any_batch(qtype):
    rng = np.random.default_rng(3)
    n, k = 40, 512
    gid = W.GGML_ID[qtype]
    w = W.quant_table(rng, n, k, qtype, (0.004, 0.012))
    x = awkward_acts(rng, 9, k)
    alone = [O.qmm(w, gid, n, k, x[j:j + 1]) for j in range(9)]
    for m in (2, 5, 9):
        batch = O.qmm(w, gid, n, k, x[:m], threads=3)
        for j in range(m):
            assert np.array_equal(batch[j].view(np.uint32), alone[j][0].view(np.uint32))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_a_weight_row_prefix_equals_the_start_of_the_product(qtype):
    rng = np.random.default_rng(17)
    gid = W.GGML_ID[qtype]
    for n, k, m, rows in [(10, 512, 3, 7), (600, 256, 2, 450), (64, 768, 5, 1)]:
        w = W.quant_table(rng, n, k, qtype, (0.004, 0.012))
        x = noise(rng, m, k, 1.0)
        whole = O.qmm(w, gid, n, k, x)
        part = O.qmm(w, gid, n, k, x, rows=rows)
        assert np.array_equal(part, whole[:, :rows])
        for bad in (0, n + 1):
            with pytest.raises(O.OracleError):
                O.qmm(w, gid, n, k, x, rows=bad)


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_zero_activations_give_exact_zeros(qtype):
    rng = np.random.default_rng(6)
    w = W.quant_table(rng, 9, 512, qtype, (0.004, 0.012))
    out = O.qmm(w, W.GGML_ID[qtype], 9, 512, np.zeros((4, 512), np.float32))
    assert np.all(out == 0.0) and not np.signbit(out).any()


def test_f16_activations_are_the_widened_values():
    rng = np.random.default_rng(8)
    n, k = 12, 256
    w = W.quant_table(rng, n, k, "q4_0", (0.004, 0.012))
    x = noise(rng, 3, k, 2.0).astype(np.float16)
    assert np.array_equal(O.qmm(w, O.Q4_0, n, k, x), O.qmm(w, O.Q4_0, n, k, x.astype(np.float32)))
