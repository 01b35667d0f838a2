//! Finds liblloom_hip.so and tells rustc to link it.
//!
//! Search order: `LLOOM_HIP_LIB_DIR` (a directory holding liblloom_hip.so),
//! then the in-tree build next to this crate (`../../lloom_amd`, where
//! `make -C lloom_amd` puts it).  The header this crate mirrors is watched so a
//! changed ABI rebuilds dependants.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=LLOOM_HIP_LIB_DIR");
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let in_tree = manifest.join("../../lloom_amd");
    let dir = match env::var_os("LLOOM_HIP_LIB_DIR") {
        Some(d) => PathBuf::from(d),
        None => in_tree,
    };
    let so = dir.join("liblloom_hip.so");
    if !so.exists() {
        panic!(
            "liblloom_hip.so not found in {} (build it with `make -C lloom_amd` or set LLOOM_HIP_LIB_DIR)",
            dir.display()
        );
    }
    let header = manifest.join("../../include/lloom_hip.h");
    println!("cargo:rerun-if-changed={}", header.display());
    println!("cargo:rerun-if-changed={}", so.display());
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=lloom_hip");
    // Let dependants' build scripts find the library too (DEP_LLOOM_HIP_LIB_DIR).
    println!("cargo:lib_dir={}", dir.display());
}
