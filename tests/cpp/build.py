"""Build the C++ GPU test of include/cuca_ops.hpp (tests/cpp/test_ops).

    python tests/cpp/build.py

Links libcuca_hip.so (the product) and liboracle.so (the CPU checker); the
run-time search path is relative to the binary, so the tree can move.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BIN = os.path.join(HERE, "test_ops")


def build(verbose=False):
    tmp = BIN + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Wno-unused-variable",
           f"-I{os.path.join(ROOT, 'include')}", os.path.join(HERE, "test_ops.cpp"),
           "-o", tmp, f"-L{os.path.join(ROOT, 'cuca_amd')}", "-lcuca_hip",
           f"-L{os.path.join(ROOT, 'oracle')}", "-l:liboracle.so",
           "-Wl,-rpath,$ORIGIN/../../cuca_amd:$ORIGIN/../../oracle", "-Wl,--no-undefined"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, BIN)
    return BIN


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
