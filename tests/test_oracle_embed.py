"""Pins the oracle's Q4_0 / Q8_0 dequant and embedding gather (CPU only).

- quants.bin golden rows (the reference's fixture, gguf-py = llama.cpp
  dequantize_row_*, 32 blocks per type at scale 1.0): bit-exact.
- The reference's closed-form KATs quant.rs:550-577 (scale 2.0 and 4.0).
- The scale folding order of quant.rs:121-123 against its alternative.
- TokenEmbedding::rows errors (quant.rs:362-374, 395-400).
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quants_legacy.npz")


def f16_bytes(v):
    return np.array([v], np.float16).view(np.uint8)


@pytest.mark.parametrize("name,ty", [("q4_0", O.Q4_0), ("q8_0", O.Q8_0)])
def test_golden_rows_bit_exact(name, ty):
    g = np.load(GOLDEN)
    blocks, expected = g[name + "_blocks"], g[name + "_expected"]
    out = O.dequant_row(ty, blocks, 1.0, expected.size)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))


def test_golden_special_blocks():
    # block 0 is zero data with d = 1.0, block 1 is 0xFF data with d = -0.75
    g = np.load(GOLDEN)
    q4 = O.dequant_row(O.Q4_0, g["q4_0_blocks"], 1.0, 1024)
    assert np.all(q4[:32] == -8.0)          # nibble 0 - 8
    assert np.all(q4[32:64] == 7 * -0.75)   # nibble 15 - 8, times d
    q8 = O.dequant_row(O.Q8_0, g["q8_0_blocks"], 1.0, 1024)
    assert np.all(q8[:32] == 0.0)
    assert np.all(q8[32:64] == 0.75)        # int8 -1 times d


def test_kat_q4_0_scale_2():
    # quant.rs:550-562: d = 0.5, byte j = j | (15 - j) << 4, scale 2.0
    block = np.concatenate([f16_bytes(0.5), np.array([j | ((15 - j) << 4) for j in range(16)],
                                                     np.uint8)])
    out = O.dequant_row(O.Q4_0, block, 2.0, 32)
    for j in range(16):
        assert out[j] == (j - 8.0) * 0.5 * 2.0
        assert out[j + 16] == ((15 - j) - 8.0) * 0.5 * 2.0


def test_kat_q8_0_two_blocks_scale_4():
    # quant.rs:564-577: d = 0.25, quants (j * 8 - 128) as i8, two blocks, scale 4.0
    quants = np.array([(j * 8 - 128) for j in range(32)], np.int64).astype(np.int8)
    block = np.concatenate([f16_bytes(0.25), quants.view(np.uint8)])
    out = O.dequant_row(O.Q8_0, np.concatenate([block, block]), 4.0, 64)
    for i in range(64):
        assert out[i] == float(quants[i % 32]) * 0.25 * 4.0


def test_scale_folds_into_d_first():
    # quant.rs:121-123: d' = f32(d) * scale, then q * d'.  With these values
    # the two orders round differently; the oracle must take the folded one.
    d, scale = np.array([10271], np.uint16).view(np.float16)[0], np.float32(16.917416)
    block = np.concatenate([np.array([d]).view(np.uint8),
                            np.full(32, 0xCF, np.uint8)])  # int8 -49
    out = O.dequant_row(O.Q8_0, block, float(scale), 32)
    folded = np.float32(-49) * (np.float32(d) * scale)
    unfolded = (np.float32(-49) * np.float32(d)) * scale
    assert folded != unfolded
    assert out[0] == folded


def test_dequant_row_rejects_bad_geometry():
    with pytest.raises(ValueError):
        O.dequant_row(O.Q4_0, np.zeros(17, np.uint8), 1.0, 32)   # quant.rs:681
    with pytest.raises(ValueError):
        O.dequant_row(O.Q8_0, np.zeros(34, np.uint8), 1.0, 48)   # not whole blocks


def test_embed_is_rows_of_dequant_and_f16_is_rne():
    rng = np.random.default_rng(5)
    vocab, hidden = 50, 96
    for ty, bs in ((O.Q4_0, 18), (O.Q8_0, 34)):
        table = rng.integers(0, 256, vocab * hidden // 32 * bs).astype(np.uint8)
        # valid finite f16 scales
        t = table.reshape(-1, bs)
        t[:, :2] = np.float16(rng.uniform(0.001, 0.05, t.shape[0])).reshape(-1, 1).view(np.uint8)
        ids = rng.integers(0, vocab, 33).astype(np.uint32)
        out = O.embed(table, ty, vocab, hidden, ids, 1.7, threads=4)
        rb = hidden // 32 * bs
        for r, i in enumerate(ids):
            row = O.dequant_row(ty, table[i * rb:(i + 1) * rb], 1.7, hidden)
            assert np.array_equal(out[r], row)
        out16 = O.embed(table, ty, vocab, hidden, ids, 1.7, out_dtype=np.float16)
        assert np.array_equal(out16.view(np.uint16), out.astype(np.float16).view(np.uint16))


def test_embed_errors_like_the_reference():
    table = np.zeros(4 * 18, np.uint8)
    with pytest.raises(O.OracleError, match="token id 4 outside the embedding table of 4 rows"):
        O.embed(table, O.Q4_0, 4, 32, np.array([0, 4], np.uint32), 1.0)
    with pytest.raises(O.OracleError, match="not a whole number"):
        O.embed(table, O.Q4_0, 4, 40, np.array([0], np.uint32), 1.0)
