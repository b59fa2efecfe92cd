// Links libgbsample_hip.so (built by `python rexl3_amd/build.py`, hipcc for gfx950). REXL3_GBS_LIB_DIR names its
// directory; the default is the repository's build output relative to this crate.
fn main() {
    let dir = std::env::var("REXL3_GBS_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR");
        format!("{here}/../../rexl3_amd/lib")
    });
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=gbsample_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=REXL3_GBS_LIB_DIR");
}
