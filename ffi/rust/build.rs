// Links the prebuilt gfx950 library.  WOHPER_HIP_LIB_DIR names the directory
// holding libwohper_hip.so (built by `python -c "import __graft_entry__ as g;
// g.build()"` into wohper_amd/); the HIP runtime it needs is found through
// the usual loader path (/opt/rocm/lib).
fn main() {
    println!("cargo:rerun-if-env-changed=WOHPER_HIP_LIB_DIR");
    if let Ok(dir) = std::env::var("WOHPER_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
    }
    println!("cargo:rustc-link-lib=dylib=wohper_hip");
}
