// Where to find libaxis_hip.so: AXIS_HIP_LIB_DIR, else the in-tree build next to this crate
// (axis_amd/, written by `python -m axis_amd.build`).  The library needs the ROCm runtime
// (libamdhip64) at run time.
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = match env::var("AXIS_HIP_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../axis_amd"),
    };
    println!("cargo:rerun-if-env-changed=AXIS_HIP_LIB_DIR");
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
}
