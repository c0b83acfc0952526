//! Links libnemotron_hip.so.  NEMOTRON_HIP_LIB_DIR names the directory that
//! holds it (the `lib/` folder `make -C nemotron-cutile-rs_amd` writes);
//! without it the in-tree build next to this crate is used.  The library
//! itself links only libamdhip64 and carries the gfx950 code object, so no
//! ROCm headers or HIP compiler are needed to build a dependent crate.
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = match env::var("NEMOTRON_HIP_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("../../nemotron-cutile-rs_amd/lib"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=nemotron_hip");
    // for this crate's own tests and examples; dependents add their own rpath or LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    println!("cargo:rerun-if-env-changed=NEMOTRON_HIP_LIB_DIR");
    println!("cargo:lib_dir={}", dir.display());
}
