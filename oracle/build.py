"""Build the CPU oracle (test infrastructure: the parity checker and the CPU
baseline timer; never part of the product path).

    python oracle/build.py

Compiles cuca_oracle.c with gcc into oracle/liboracle.so.  -ffp-contract=off
keeps every f32 product and sum individually rounded, as Rust (which never
contracts to FMA) and candle's scalar kernels do.

The reference itself (nassor/cuca, Rust + candle 0.11.1) cannot be built in
this image: there is no cargo/rustc and candle is not vendored, so there is
no oracle/_ref build.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    src = os.path.join(HERE, "cuca_oracle.c")
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-D_GNU_SOURCE", "-ffp-contract=off",
           "-fno-fast-math", "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra",
           "-Wno-unused-parameter", src, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
