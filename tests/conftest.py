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


@pytest.fixture(autouse=True)
def _name_the_test(request):
    """Tag the raw-error records of assert_close with the running test."""
    import helpers
    helpers.CURRENT_TEST[0] = request.node.nodeid
    yield


def pytest_terminal_summary(terminalreporter):
    """The unfloored errors behind the tolerance bars: per op family (test
    file), the maximum relative error (f32) and f16 ulps, how many
    elements passed only through a stated floor, and how many expected
    values were NaN or inf (each matched by value, not by a tolerance)."""
    try:
        import helpers
    except ImportError:
        return
    if not helpers.RAW:
        return
    fam = {}
    for test, what, st in helpers.RAW:
        key = (test.split("::")[0].split("/")[-1], st["dtype"])
        f = fam.setdefault(key, {"n": 0, "worst": 0.0, "floored": 0, "nonfinite": 0, "at": ""})
        v = st.get("max_rel", st.get("max_ulp", 0.0))
        f["n"] += st["n"]
        f["floored"] += st["floored"]
        f["nonfinite"] += st.get("nonfinite", 0)
        if v > f["worst"]:
            f["worst"], f["at"] = v, f"{test.split('::')[-1]} {what}"
    tr = terminalreporter
    tr.section("raw errors before floors (f32: max relative error; f16: max ulps)")
    for (file, dt), f in sorted(fam.items()):
        unit = "rel" if dt == "f32" else "ulp"
        tr.write_line(f"{file:28s} {dt}  max {unit} {f['worst']:.3g}  values {f['n']}  "
                      f"within the bar only by a floor {f['floored']}  "
                      f"expected NaN/inf (matched by value) {f['nonfinite']}  (worst: {f['at']})")
