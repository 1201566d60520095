//! Links libg4attn.so (`make -C gemma4-rs_amd`: hipcc --offload-arch=gfx950),
//! the only library the crate binds; it brings the HIP runtime in itself.
//! `G4ATTN_LIB_DIR` names the directory that holds it (default: `../lib`,
//! beside this crate in gemma4-rs_amd).

use std::env;
use std::path::PathBuf;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let lib_dir = env::var("G4ATTN_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join("lib"));
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=g4attn");
    // This package's test binaries find the library where it was linked
    // from; Cargo does not pass link arguments on to dependent crates.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-env-changed=G4ATTN_LIB_DIR");
    println!("cargo:rerun-if-changed=build.rs");
}
