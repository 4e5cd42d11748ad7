"""Build libcuca_hip.so: the gfx950 code object plus the C-ABI host runtime.

    python -m cuca_amd.build

1. hipcc compiles csrc/kernels/cuca_kernels.hip for gfx950 only into a raw
   ELF code object (_build/cuca_kernels.co), with -ffp-contract=off (RoPE
   and the dequant are bit-exact only without FMA contraction) and packed
   FP32 instructions disabled.
2. The kernel names in csrc/kernel_list.inc are checked against the code
   object's symbols.
3. hipcc compiles csrc/noalloc.hip (host and gfx950 device code: the
   allocation-free entry points' scratch array, a registered __device__
   variable) into a position-independent object.
4. g++ compiles csrc/runtime.cpp (host code only) with the code object
   embedded (.incbin) and links it with that object into libcuca_hip.so,
   linked to libamdhip64.

Both outputs are written in-tree (cuca_amd/), so the .so travels with the
repository snapshot to the GPU box; nothing is JIT-compiled at run time.
"""

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcuca_hip.so")
CODE_OBJECT = os.path.join(BUILD, "cuca_kernels.co")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "--offload-device-only", "--no-gpu-bundle-output",
    "-O3", "-std=c++17", "-ffp-contract=off", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Werror=return-type",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise
    noise = re.compile(r"packed-fp32-ops|^\d+ warnings? generated")
    err = "\n".join(l for l in res.stderr.splitlines() if not noise.search(l))
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def kernel_names():
    names = []
    with open(os.path.join(CSRC, "kernel_list.inc")) as f:
        for line in f:
            m = re.match(r"\s*K\((\w+)\)", line)
            if m:
                names.append(m.group(1))
    return names


def code_object_kernels(path):
    out = subprocess.run([os.path.join(ROCM, "llvm/bin/llvm-readelf"), "--symbols", path],
                         capture_output=True, text=True, check=True).stdout
    syms = set()
    for line in out.splitlines():
        parts = line.split()
        if parts and parts[-1].endswith(".kd"):  # one kernel descriptor per kernel
            syms.add(parts[-1][:-3])
    return syms


def kernel_code_sha256(name, path=CODE_OBJECT):
    """SHA-256 of one kernel's machine code in the code object (its function
    symbol's bytes in the ELF), or None when the object or the symbol is
    missing.  A measurement recorded against a kernel names this hash, so
    it can be recognised as stale once the kernel's code changes."""
    import hashlib
    import struct
    try:
        with open(path, "rb") as f:
            elf = f.read()
    except OSError:
        return None
    if elf[:4] != b"\x7fELF" or elf[4] != 2:  # 64-bit ELF
        return None
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    for sec in secs:
        if sec[1] != 2:  # SHT_SYMTAB
            continue
        strtab = secs[sec[6]]
        for off in range(sec[4], sec[4] + sec[5], sec[9]):
            st_name, st_info, _, st_shndx, st_value, st_size = struct.unpack_from("<IBBHQQ", elf, off)
            start = strtab[4] + st_name
            end = elf.index(b"\0", start)
            if elf[start:end].decode() != name or (st_info & 0xF) != 2 or st_shndx >= shnum:  # STT_FUNC
                continue
            text = secs[st_shndx]
            pos = text[4] + (st_value - text[3])  # file offset: sh_offset + (value - sh_addr)
            return hashlib.sha256(elf[pos:pos + st_size]).hexdigest()
    return None


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    co_tmp = CODE_OBJECT + ".tmp"
    _run([os.path.join(ROCM, "bin/hipcc"), *HIPCC_FLAGS,
          os.path.join(CSRC, "kernels", "cuca_kernels.hip"), "-o", co_tmp], verbose)
    os.replace(co_tmp, CODE_OBJECT)
    listed = kernel_names()
    present = code_object_kernels(CODE_OBJECT)
    missing = [k for k in listed if k not in present]
    unlisted = sorted(present - set(listed))
    if missing or unlisted:
        raise RuntimeError(f"kernel_list.inc and the code object disagree: missing {missing}, "
                           f"unlisted {unlisted}")
    noalloc_obj = os.path.join(BUILD, "noalloc.o")
    _run([os.path.join(ROCM, "bin/hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall",
          f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", "-c",
          os.path.join(CSRC, "noalloc.hip"), "-o", noalloc_obj], verbose)
    lib_tmp = LIB + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", f"-DCUCA_CODE_OBJECT=\"{CODE_OBJECT}\"",
          f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", f"-I{ROCM}/include",
          os.path.join(CSRC, "runtime.cpp"), noalloc_obj, "-o", lib_tmp,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
          "-Wl,--no-undefined"], verbose)
    os.replace(lib_tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
