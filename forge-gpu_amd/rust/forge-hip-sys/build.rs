// Link libforge_hip.so (built by `python forge-gpu_amd/build.py`) and the HIP runtime.
//
// FORGE_HIP_LIB_DIR overrides the directory of libforge_hip.so (default: forge-gpu_amd/lib,
// two levels above this crate); ROCM_PATH the ROCm install (default /opt/rocm) whose lib/ holds
// libamdhip64.so.
use std::env;
use std::path::PathBuf;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let lib_dir = env::var("FORGE_HIP_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join("..").join("lib"));
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=forge_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // the library is found at run time next to where it was built
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-env-changed=FORGE_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
