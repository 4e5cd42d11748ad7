import os
import sys

import pytest

# torch ships its own HIP runtime with the SONAME libamdhip64.so.7.  Loading
# it first makes the dynamic loader bind libcuca_hip.so to that same runtime,
# so one process never holds two HIP runtimes (the second one would see no
# device).  Tests that use torch tensors as device buffers rely on this.
try:
    import torch  # noqa: F401
except Exception:  # torch is optional for the CPU tests
    torch = None

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ctx():
    """One cuca_hip context on device 0 for the whole GPU session."""
    from cuca_amd import hip
    c = hip.Context(0)
    yield c
    c.close()
