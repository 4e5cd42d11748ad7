"""Pins the oracle's binary16 conversions (CPU only): the `half` crate's
f16 -> f32 is exact and f32 -> f16 rounds to nearest-even.  Both the scalar
restatement and the bulk path the oracle's ops use (x86 F16C when the CPU
has it) are checked against numpy: every one of the 65536 f16 patterns, and
f32 patterns covering every exponent, the rounding ties, the f16 subnormal
range, overflow, infinities and NaNs.
"""
import numpy as np

from oracle import oracle as O


def _h2f(fn, h):
    out = np.empty(h.shape, np.float32)
    fn(h.ctypes.data, out.ctypes.data, h.size)
    return out


def _f2h(fn, f):
    out = np.empty(f.shape, np.uint16)
    fn(f.ctypes.data, out.ctypes.data, f.size)
    return out


def test_every_f16_widens_exactly_on_both_paths():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    L = O.lib()
    for fn in (L.oracle_f16_to_f32_n, L.oracle_f16_to_f32_soft_n):
        got = _h2f(fn, h)
        nan = np.isnan(want)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
        assert np.all(np.isnan(got[nan]))


def f32_patterns():
    rng = np.random.default_rng(0)
    bits = [rng.integers(0, 1 << 32, 3_000_000, dtype=np.uint64).astype(np.uint32)]
    # every exponent of the f16 range and around it, with mantissas that
    # land on, just below and just above the rounding midpoints
    e = np.arange(96, 160, dtype=np.uint32)
    tails = np.array([0, 1, 0xfff, 0x1000, 0x1001, 0x1fff, 0x2000, 0x3000, 0x7fe000, 0x7fefff,
                      0x7ff000, 0x7fffff], np.uint32)
    m = (rng.integers(0, 1 << 10, (e.size, 40), dtype=np.uint32) << 13)[..., None] | tails
    bits.append(((e[:, None, None] << 23) | m).reshape(-1))
    bits.append(np.array([0, 0x7f800000, 0x7fc00000, 0x7f800001, 0x477fe000, 0x477fefff,
                          0x477ff000, 0x33000000, 0x33000001, 0x32ffffff], np.uint32))
    b = np.concatenate(bits)
    return np.concatenate([b, b | 0x80000000]).view(np.float32)


def test_f32_rounds_to_nearest_even_on_both_paths():
    f = f32_patterns()
    with np.errstate(over="ignore", invalid="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    L = O.lib()
    for fn in (L.oracle_f32_to_f16_n, L.oracle_f32_to_f16_soft_n):
        got = _f2h(fn, f)
        assert np.array_equal(got[~nan], want[~nan])
        assert np.all(np.isnan(got[nan].view(np.float16)))


def test_bulk_path_tails():
    """Lengths that are not multiples of the 8-wide hardware step."""
    L = O.lib()
    rng = np.random.default_rng(1)
    for n in (1, 7, 8, 9, 15, 17):
        f = rng.standard_normal(n).astype(np.float32) * 1000
        assert np.array_equal(_f2h(L.oracle_f32_to_f16_n, f), f.astype(np.float16).view(np.uint16))
        h = f.astype(np.float16).view(np.uint16)
        assert np.array_equal(_h2f(L.oracle_f16_to_f32_n, h), h.view(np.float16).astype(np.float32))
