//! Builds libnomas_moe.so with the package's own Makefile (hipcc,
//! --offload-arch=gfx950) and links it.  The crate sits at
//! hy-nomas-rs_amd/rust/nomas-moe-sys, so the package is two levels up; set
//! NOMAS_MOE_PKG to build from another checkout.
use std::{env, path::PathBuf, process::Command};

fn main() {
    let pkg = match env::var("NOMAS_MOE_PKG") {
        Ok(p) => PathBuf::from(p),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../.."),
    };
    let pkg = pkg.canonicalize().expect("the hy-nomas-rs_amd package directory");
    let jobs = env::var("NUM_JOBS").unwrap_or_else(|_| "8".into());
    let status = Command::new("make")
        .arg("-C")
        .arg(&pkg)
        .arg("-j")
        .arg(&jobs)
        .arg("libnomas_moe.so")
        .status()
        .expect("running make");
    assert!(status.success(), "building libnomas_moe.so (hipcc --offload-arch=gfx950) failed");
    println!("cargo:rustc-link-search=native={}", pkg.display());
    println!("cargo:rustc-link-lib=dylib=nomas_moe");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", pkg.display());
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
    println!("cargo:rerun-if-changed={}", pkg.join("../include/nomas_moe.h").display());
    println!("cargo:rerun-if-env-changed=NOMAS_MOE_PKG");
}
