// Links the prebuilt libvelox_hip.so (built for gfx950 by
// `python velox_amd/build.py`; no Python is needed at run time) and the HIP
// runtime it uses.  VELOX_HIP_LIB_DIR names the folder of the library;
// ROCM_PATH (default /opt/rocm) that of libamdhip64.
fn main() {
    let dir = std::env::var("VELOX_HIP_LIB_DIR")
        .expect("set VELOX_HIP_LIB_DIR to the folder that holds libvelox_hip.so");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=velox_hip");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=VELOX_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
