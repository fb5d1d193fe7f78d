// Links libark_opt.so (built by `make -C ark_amd/csrc`) and the HIP runtime.
// ARK_OPT_LIB_DIR overrides the library's directory (default: the
// repository's ark_amd/lib); ROCM_PATH the ROCm root (default /opt/rocm).
use std::env;
use std::path::PathBuf;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let lib_dir = env::var("ARK_OPT_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../lib"));
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=ark_opt");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=ARK_OPT_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
