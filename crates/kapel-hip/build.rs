//! Links libkapel_hip.so (built by `python -m kapel_amd.build`, or by hipcc
//! on kapel_amd/csrc) and the HIP runtime when the `hip` feature is on.
//!
//! KAPEL_HIP_LIB_DIR: the directory of libkapel_hip.so (default: the
//! `kapel_amd` directory of a kapel-hip checkout beside this crate).
//! ROCM_PATH: the ROCm installation (default /opt/rocm), for libamdhip64.

use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=KAPEL_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    if env::var_os("CARGO_FEATURE_HIP").is_none() {
        return;
    }
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("set by cargo"));
    let lib_dir = env::var_os("KAPEL_HIP_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|| manifest.join("../../kapel_amd"));
    let rocm = env::var_os("ROCM_PATH").map_or_else(|| PathBuf::from("/opt/rocm"), PathBuf::from);
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}", rocm.join("lib").display());
    println!("cargo:rustc-link-lib=dylib=kapel_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // Found at run time without LD_LIBRARY_PATH.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
}
