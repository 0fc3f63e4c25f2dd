// Links libbdh_hip.so, built by `python -m burn_dragon_amd.build` (hipcc,
// gfx950).  BDH_HIP_LIB_DIR names its directory; by default the
// burn_dragon_amd package directory two levels above this crate.
fn main() {
    let dir = std::env::var("BDH_HIP_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR");
        format!("{here}/../../burn_dragon_amd")
    });
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=bdh_hip");
    println!("cargo:rerun-if-env-changed=BDH_HIP_LIB_DIR");
}
