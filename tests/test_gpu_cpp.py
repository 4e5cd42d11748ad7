"""The C++ host side (include/cuca_ops.hpp) on the GPU: TokenEmbedding::rows,
add_rms / rms, Glu, RopeSpec::tables + apply_rope and the error mapping,
against the oracle (tests/cpp/test_ops.cpp, built by __graft_entry__.build)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_ops")


def test_cpp_host_side():
    assert os.path.exists(BIN), "tests/cpp/test_ops is not built: run __graft_entry__.build()"
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all ok" in res.stdout
