// prism-ffi/build.rs -- links libprism_hip when the `hip-dispatch` feature is
// on (prism-ffi/Cargo.toml: `hip-dispatch = []`; the crate also needs
// crate-type ["staticlib", "rlib"] so that the engine crate can use its `hip`
// module).  PRISM_HIP_LIB_DIR names the directory of libprism_hip.so (built
// by `make -C prism-engine_amd/csrc`), ROCM_PATH the ROCm install that
// provides libamdhip64.
fn main() {
    println!("cargo:rerun-if-env-changed=PRISM_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    if std::env::var_os("CARGO_FEATURE_HIP_DISPATCH").is_none() {
        return;
    }
    let lib = std::env::var("PRISM_HIP_LIB_DIR").unwrap_or_else(|_| "../prism-engine_amd".to_string());
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={lib}");
    println!("cargo:rustc-link-lib=dylib=prism_hip");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
