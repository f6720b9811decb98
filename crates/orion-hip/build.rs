// Links liborion_hip.so.  The library itself is compiled by its own build
// script (orionserve-rs_amd/build.py, hipcc for gfx950); this crate only
// emits the link line.  ORION_HIP_LIB_DIR names the directory holding it.
fn main() {
    let dir = std::env::var("ORION_HIP_LIB_DIR")
        .expect("set ORION_HIP_LIB_DIR to the directory holding liborion_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=orion_hip");
    println!("cargo:rerun-if-env-changed=ORION_HIP_LIB_DIR");
}
