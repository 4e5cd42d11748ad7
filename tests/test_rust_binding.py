"""The Rust binding crate (rust/cuca-hip-sys) against include/cuca_hip.h, on
the CPU: there is no Rust toolchain in this image, so the binding is held to
the header by reading both.

- Every function the header declares is in the `extern "C"` block of
  src/lib.rs, and nothing else is, with the same argument names, count and
  types (each C type mapped to its Rust FFI type), and the same return type.
- The #[repr(C)] structs have the header's fields, in order, with the
  mapped types, and the C layout of those types gives the offsets and size
  that the C compiler gives (measured through ctypes).
- The status, dtype, activation and RoPE-kind constants and the #defines
  carry the header's values.
- Every raw call the safe wrapper (src/safe.rs) makes exists.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cuca_hip.h")
CRATE = os.path.join(ROOT, "rust", "cuca-hip-sys")

C_TO_RUST = {
    "int64_t": "i64", "int32_t": "i32", "uint32_t": "u32", "uint64_t": "u64", "int8_t": "i8",
    "uint8_t": "u8", "float": "f32", "double": "f64", "size_t": "usize", "int": "c_int",
    "void": "c_void", "char": "c_char",
    "cuca_status": "cuca_status", "cuca_dtype": "cuca_dtype", "cuca_act": "cuca_act",
    "cuca_rope_kind": "cuca_rope_kind", "cuca_hip_ctx": "cuca_hip_ctx",
    "cuca_hip_graph": "cuca_hip_graph", "cuca_rope_spec": "cuca_rope_spec",
    "cuca_hip_kernel_time": "cuca_hip_kernel_time",
}


def rust_type(ctype):
    c = " ".join(ctype.split())
    const = c.startswith("const ")
    base = c.replace("const ", "").replace("*", "").strip()
    stars = c.count("*")
    t = C_TO_RUST[base]
    if stars == 0:
        return t
    if stars == 1:
        return ("*const " if const else "*mut ") + t
    assert stars == 2, c
    return "*mut *mut " + t


def header_text():
    return re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)


def header_functions():
    text = re.sub(r"#.*", "", header_text())
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(cuca_hip_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
        params = []
        args = " ".join(args.split())
        if args and args != "void":
            for a in args.split(","):
                m = re.match(r"(.*?)([A-Za-z_]\w*)$", a.strip())
                params.append((m.group(2), rust_type(m.group(1))))
        ret = " ".join(ret.split())
        out[name] = (None if ret == "void" else rust_type(ret), params)
    return out


def rust_functions():
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = src[src.index('extern "C" {'):]
    out = {}
    for name, args, ret in re.findall(r"pub fn (cuca_hip_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            n, t = a.split(":", 1)
            params.append((n.strip().removeprefix("r#"), " ".join(t.split())))
        out[name] = (None if not ret else " ".join(ret.split()), params)
    return out


def test_every_function_matches_the_header():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 50
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, (ret, params) in h.items():
        rret, rparams = r[name]
        assert rret == ret, (name, ret, rret)
        assert len(rparams) == len(params), (name, params, rparams)
        for (cn, ct), (rn, rt) in zip(params, rparams):
            assert cn == rn and ct == rt, (name, cn, ct, rn, rt)


def c_struct(name):
    body = dict((n, b) for b, n in re.findall(r"typedef struct \{([^{}]*)\}\s*(\w+)\s*;", header_text()))[name]
    fields = []
    for decl in body.split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        m2 = re.match(r"(.*?)([A-Za-z_]\w*(?:\s*,\s*[A-Za-z_]\w*)*)$", decl)
        ctype, names = m2.group(1).strip(), m2.group(2)
        for n in [x.strip() for x in names.split(",")]:
            fields.append((n, rust_type(ctype)))
    return fields


def rust_struct(name):
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    m = re.search(r"#\[repr\(C\)\]\s*(?:#\[derive\([^\]]*\)\]\s*)?pub struct " + name + r" \{(.*?)\}", src, re.S)
    return [(n, " ".join(t.split())) for n, t in re.findall(r"pub (\w+):\s*([^,]+),", m.group(1))]


RUST_LAYOUT = {"i32": (4, 4), "i64": (8, 8), "f32": (4, 4), "f64": (8, 8), "u32": (4, 4), "usize": (8, 8)}


def rust_offsets(fields):
    off, offs, align = 0, [], 1
    for _, t in fields:
        size, al = (8, 8) if t.startswith("*") else RUST_LAYOUT[t]
        off = (off + al - 1) // al * al
        offs.append(off)
        off += size
        align = max(align, al)
    return offs, (off + align - 1) // align * align


@pytest.mark.parametrize("name", ["cuca_rope_spec", "cuca_hip_kernel_time"])
def test_structs_match_the_header_and_the_c_layout(name):
    from cuca_amd import hip
    cf, rf = c_struct(name), rust_struct(name)
    assert cf == rf, (cf, rf)
    cty = {"cuca_rope_spec": hip.RopeSpecC, "cuca_hip_kernel_time": hip.KernelTime}[name]
    # the ctypes mirror has the header's fields in order
    assert [f[0] for f in cty._fields_] == [n for n, _ in cf]
    offs, size = rust_offsets(rf)
    assert offs == [getattr(cty, n).offset for n, _ in cf]
    assert size == ctypes.sizeof(cty)


def test_constants_match_the_header():
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    rust = {n: v for n, v in re.findall(r"pub const (CUCA_\w+): [\w:]+ = ([^;]+);", src)}
    text = header_text()
    want = {}
    for body in re.findall(r"typedef enum \{(.*?)\}", text, re.S):
        for n, v in re.findall(r"(CUCA_\w+)\s*=\s*(\d+)", body):
            want[n] = int(v)
    for n, v in re.findall(r"#define (CUCA_\w+) \(?([0-9xa-fA-Fu <]+)\)?", text):
        want[n] = eval(v.replace("u", "").strip())
    want.pop("CUCA_HIP_H", None)
    for n, v in want.items():
        assert n in rust, n
        assert eval(rust[n].replace("_", "")) == v, (n, rust[n], v)


def test_safe_wrapper_calls_exist_and_cargo_files_are_there():
    names = set(rust_functions())
    safe = open(os.path.join(CRATE, "src", "safe.rs")).read()
    used = set(re.findall(r"\b(cuca_hip_\w+)\s*[\(,}\s]", safe)) - {"cuca_hip_ctx", "cuca_hip_graph"}
    assert used and used <= names, sorted(used - names)
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "cuca-hip-sys"' in toml and 'links = "cuca_hip"' in toml
    assert "rustc-link-lib=dylib=cuca_hip" in open(os.path.join(CRATE, "build.rs")).read()
