// Link libcpb_moe.so (built in-tree by `python -m cpubrrr_amd.build`) and the
// HIP runtime it depends on.  CPB_MOE_LIB_DIR overrides the library folder;
// ROCM_PATH (default /opt/rocm) locates libamdhip64.
use std::env;
use std::path::PathBuf;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let default_dir = manifest.join("../../cpubrrr_amd");
    let lib_dir = env::var("CPB_MOE_LIB_DIR").map(PathBuf::from).unwrap_or(default_dir);
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=cpb_moe");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // the engine binary finds the library at run time without LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-env-changed=CPB_MOE_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed=../../include/cpb_moe.h");
    println!("cargo:rerun-if-changed=../../include/cpb_gguf.h");
    println!("cargo:rerun-if-changed=../../include/cpb_head.h");
}
