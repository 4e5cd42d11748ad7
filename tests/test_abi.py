"""The C ABI library on the CPU: it loads, exports every entry point
include/cuca_hip.h declares, carries a gfx950-only code object, and its
host-side pieces (RoPE tables, argument checks) behave without a GPU."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from cuca_amd import build, hip
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cuca_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cuca_hip_\w+)\s*\(", text)))


def test_every_declared_entry_point_is_exported_and_bound():
    names = declared()
    assert len(names) >= 20
    L = ctypes.CDLL(hip.LIB_PATH)
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(hip.SIGNATURES)


def test_code_object_is_gfx950_only_and_lists_every_kernel():
    assert os.path.exists(build.CODE_OBJECT)
    notes = subprocess.run([os.path.join(build.ROCM, "llvm/bin/llvm-readelf"), "--notes",
                            build.CODE_OBJECT], capture_output=True, text=True, check=True).stdout
    targets = set(re.findall(r"amdhsa\.target:\s*(\S+)", notes))
    assert targets and all(t.strip("'\"").startswith("amdgcn-amd-amdhsa--gfx950") for t in targets)
    assert set(build.kernel_names()) == build.code_object_kernels(build.CODE_OBJECT)
    # no kernel spills to scratch
    assert "private_segment_fixed_size: 0" in notes
    sizes = [int(s) for s in re.findall(r"\.private_segment_fixed_size:\s*(\d+)", notes)]
    assert sizes and max(sizes) == 0


@pytest.mark.parametrize("spec", [
    dict(n_dims=128, base=1e6, positions=64),
    dict(n_dims=128, base=5e5, positions=8192),
    dict(n_dims=256, base=1e4, positions=300),
    dict(n_dims=64, base=1e4, positions=100, freq_scale=0.25, yarn=(1.0, 32.0, 1.0, 4096)),
    dict(n_dims=16, base=1e4, positions=50, freq_scale=0.5, attn_factor=1.25),
    dict(n_dims=8, base=1e4, positions=20, factors=[1.0, 2.0, 1e30, 0.5]),
])
def test_rope_tables_bit_identical_to_the_oracle(spec):
    kw = dict(spec)
    n_dims, base, positions = kw.pop("n_dims"), kw.pop("base"), kw.pop("positions")
    c1, s1 = hip.rope_tables(hip.ROPE_NEOX, n_dims, base, positions, **kw)
    c2, s2 = O.rope_tables(n_dims, base, positions, **kw)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_rope_tables_reject_bad_specs():
    with pytest.raises(hip.CucaError, match="even"):
        hip.rope_tables(hip.ROPE_NEOX, 7, 1e4, 4)
    with pytest.raises(hip.CucaError, match="finite and positive"):
        hip.rope_tables(hip.ROPE_NEOX, 4, 1e4, 4, factors=[1.0, 0.0])


def test_context_without_a_gfx950_reports_an_error():
    p = ctypes.c_void_p()
    L = hip.lib()
    st = L.cuca_hip_ctx_create(0, ctypes.byref(p))
    if st == hip.OK:  # running on the GPU box
        L.cuca_hip_ctx_destroy(p.value)
        return
    assert st in (hip.HIP_ERROR, hip.NOT_GFX950)
    assert p.value is None
    assert L.cuca_hip_last_error(None)


def test_ops_validate_on_the_host_before_any_device_work():
    from cuca_amd import ops
    with pytest.raises(hip.CucaError, match="not a whole number of Q4_0 blocks"):
        ops.TokenEmbedding(None, hip.GGML_Q4_0, np.zeros(18, np.uint8), 1, 40)
    with pytest.raises(hip.CucaError, match="do not hold 2 rows"):
        ops.TokenEmbedding(None, hip.GGML_Q4_0, np.zeros(18, np.uint8), 2, 32)



def test_kv_slots_place_rows_where_store_rows_does():
    rng = np.random.default_rng(5)
    n_kv, d = 3, 4
    for table, start, t in [([5, 0, 9, 2], 0, 64), ([5, 0, 9, 2], 13, 40), ([7], 3, 1),
                            ([1, 2], 15, 2)]:
        slots = hip.kv_slots(table, start, t, 10)
        src = rng.standard_normal((n_kv, t, d)).astype(np.float32)
        want = np.zeros((10, n_kv, 16, d), np.float32)
        O.store_rows(table, start, src, want)
        got = np.zeros_like(want)
        got[slots // 16, :, slots % 16, :] = src.transpose(1, 0, 2)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("table,start,t,where", [
    ([3, hip.NO_BLOCK], 0, 20, 16), ([3], 10, 10, 16), ([3, 10], 0, 20, 16)])
def test_kv_slots_reject_positions_without_a_block(table, start, t, where):
    with pytest.raises(hip.CucaError, match=f"position {where} has no K/V block "
                       r"\(it left the window or was never allocated\)"):
        hip.kv_slots(table, start, t, 10)


def test_kernels_bit_cast_no_vector_element_lvalue():
    # hipcc (ROCm 7.2) compiled __builtin_bit_cast(T, v.y) of an ext-vector
    # element to a read of element 0; the kernels cast whole vectors or
    # values passed through a scalar instead
    kdir = os.path.join(ROOT, "cuca_amd", "csrc", "kernels")
    pat = re.compile(r"__builtin_bit_cast\([^,()]+,\s*[\w\[\]]+\.[xyzw]\s*\)")
    for f in os.listdir(kdir):
        text = open(os.path.join(kdir, f)).read()
        text = re.sub(r"//[^\n]*", "", text)
        assert not pat.search(text), (f, pat.search(text).group(0))
