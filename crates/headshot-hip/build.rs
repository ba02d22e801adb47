//! Links libheadshot_hip.so (built by `python -m headshot_amd.build`, which
//! runs hipcc --offload-arch=gfx950) and the ROCm HIP runtime it uses for
//! allocation and streams.
use std::env;
use std::path::PathBuf;

fn main() {
    // <repo>/crates/headshot-hip -> <repo>/headshot_amd, unless overridden
    let lib_dir = env::var("HEADSHOT_HIP_LIB_DIR").map(PathBuf::from).unwrap_or_else(|_| {
        PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../headshot_amd")
    });
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=headshot_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=HEADSHOT_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
