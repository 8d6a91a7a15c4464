// Links libhuncho_rocm.so. HUNCHO_ROCM_LIB_DIR points at the directory that holds it (the
// repository's huncho_amd/_build after `python -m huncho_amd.build`); the ROCm runtime it needs
// (libamdhip64, libhipblaslt) is found through the library's own rpath.
fn main() {
    let dir = std::env::var("HUNCHO_ROCM_LIB_DIR").unwrap_or_else(|_| "/opt/huncho/lib".into());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=huncho_rocm");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=HUNCHO_ROCM_LIB_DIR");
}
