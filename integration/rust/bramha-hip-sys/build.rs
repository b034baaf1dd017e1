//! Link libbramha_hip.so (built by `python bramha_amd/build.py`) and the HIP runtime.
//! BRAMHA_HIP_LIB_DIR: directory of libbramha_hip.so (default: ../../../bramha_amd, the in-tree
//! build next to this crate); ROCM_PATH: the ROCm install (default /opt/rocm).
use std::env;
use std::path::PathBuf;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let lib_dir = env::var("BRAMHA_HIP_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../../bramha_amd"));
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=bramha_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // the library is loaded from where it was built
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-env-changed=BRAMHA_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed={}", lib_dir.join("libbramha_hip.so").display());
}
