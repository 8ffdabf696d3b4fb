// Tells rustc where libqe.so is: $QE_LIB_DIR, else the package directory the library is built in
// (../../mac-gpu-compiler_amd relative to this crate).
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = match env::var("QE_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../../mac-gpu-compiler_amd"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=qe");
    println!("cargo:rerun-if-env-changed=QE_LIB_DIR");
}
