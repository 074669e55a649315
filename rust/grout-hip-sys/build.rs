//! Links libgrout_attn_hip.so.  The library is built by
//! `python -m grout_amd.build` into `grout_amd/`; point GROUT_AMD_LIB_DIR at
//! another directory to link a copy installed elsewhere.
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = match env::var("GROUT_AMD_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../grout_amd"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=grout_attn_hip");
    // The HIP runtime the library itself links against.
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=GROUT_AMD_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed=../../include/grout_attn_hip.h");
}
