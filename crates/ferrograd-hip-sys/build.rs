//! Links libferrograd_hip.so.  The library is built by
//! `python -m ferrograd_amd._build` (hipcc, gfx950) into `ferrograd_amd/` of
//! this repository; FERROGRAD_HIP_LIB_DIR overrides where it is found.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=FERROGRAD_HIP_LIB_DIR");
    let dir = match env::var("FERROGRAD_HIP_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => {
            let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
            manifest.join("..").join("..").join("ferrograd_amd")
        }
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=ferrograd_hip");
    // The HIP runtime the library links against.
    println!("cargo:rustc-link-search=native=/opt/rocm/lib");
}
