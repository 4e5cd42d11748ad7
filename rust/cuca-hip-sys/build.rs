//! Link libcuca_hip.so: built in-tree by `python -m cuca_amd.build` into
//! `cuca_amd/` of this repository (CUCA_HIP_LIB_DIR overrides the search
//! directory).  The library depends on libamdhip64 only (ROCm's HIP
//! runtime, found through the rpath the build records).
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = env::var("CUCA_HIP_LIB_DIR").map(PathBuf::from).unwrap_or_else(|_| {
        PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../cuca_amd")
    });
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=cuca_hip");
    println!("cargo:rerun-if-env-changed=CUCA_HIP_LIB_DIR");
    println!("cargo:rerun-if-changed=../../include/cuca_hip.h");
}
