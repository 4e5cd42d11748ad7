"""Extract the Q4_0 and Q8_0 golden rows from the reference's quants.bin.

    python tests/golden/make_quants_fixture.py [path/to/quants.bin]

Reads the data file src/provider/local/testdata/quants/quants.bin of
nassor/cuca (written by its make_fixture.py from gguf-py's
`quants.dequantize`, which mirrors llama.cpp's `dequantize_row_*`) and keeps
the two entries this build decodes: ggml type 2 (Q4_0) and 8 (Q8_0), 32
blocks each (a zero-data block, a 0xFF block, 30 random blocks; seed 0xC0CA)
with their expected f32 values at scale 1.0.  Layout of quants.bin, as its
consumer reads it (model/quant/format_tests.rs:40-80): magic "CQF1", u32
entry count; per entry u32 type, u32 blocks, u32 scales, the blocks, then
per scale f32 scale, u8 kind (0: blocks*32 f32 values follow; 1: an FNV-1a
64-bit hash follows).

Writes tests/golden/quants_legacy.npz (uint8 blocks, float32 expected) —
data only; nothing from the reference's code is copied.
"""

import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT = "/root/reference/src/provider/local/testdata/quants/quants.bin"
# (values per block, bytes per block), testdata/quants/sizes.txt
SIZES = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84),
         11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
         16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18),
         21: (256, 110), 22: (256, 82), 23: (256, 136), 29: (256, 56), 34: (256, 54),
         35: (256, 66), 39: (32, 17), 40: (64, 36)}
KEEP = {2: "q4_0", 8: "q8_0"}


def main(path):
    data = open(path, "rb").read()
    assert data[:4] == b"CQF1", "not a CQF1 fixture"
    (n,) = struct.unpack_from("<I", data, 4)
    at = 8
    out = {}
    for _ in range(n):
        ty, blocks, n_scales = struct.unpack_from("<III", data, at)
        at += 12
        bs, ts = SIZES[ty]
        raw = data[at:at + blocks * ts]
        at += blocks * ts
        for _ in range(n_scales):
            scale, kind = struct.unpack_from("<fB", data, at)
            at += 5
            if kind == 0:
                vals = np.frombuffer(data, "<f4", blocks * bs, at).copy()
                at += blocks * bs * 4
            else:
                vals = None
                at += 8
            if ty in KEEP and kind == 0 and scale == 1.0:
                out[KEEP[ty] + "_blocks"] = np.frombuffer(raw, np.uint8).copy()
                out[KEEP[ty] + "_expected"] = vals
    assert at == len(data), "trailing bytes: layout mismatch"
    assert set(out) == {"q4_0_blocks", "q4_0_expected", "q8_0_blocks", "q8_0_expected"}
    dst = os.path.join(HERE, "quants_legacy.npz")
    np.savez(dst, **out)
    for k, v in out.items():
        print(k, v.dtype, v.shape)
    print("wrote", dst)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else DEFAULT)
