//! Link step only: points rustc at the prebuilt libwrs_attn.so. The HIP
//! sources are compiled by their own Makefile (hipcc, gfx950), never here.
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = match env::var("WRS_ATTN_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        // default: the library built in place in this repository
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap())
            .join("../../whisper.rs_amd/lib"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=wrs_attn");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
    println!("cargo:rerun-if-env-changed=WRS_ATTN_LIB_DIR");
}
