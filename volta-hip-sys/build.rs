//! Builds libvolta_hip.so with hipcc (through the library's Makefile) and links it.
//! VOLTA_HIP_ROOT points at this repository's checkout (default: the crate's parent).
use std::path::PathBuf;
use std::process::Command;

fn main() {
    let root = std::env::var("VOLTA_HIP_ROOT").map(PathBuf::from).unwrap_or_else(|_| {
        PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR")).join("..")
    });
    let csrc = root.join("volta_amd").join("csrc");
    let status = Command::new("make")
        .arg("-C")
        .arg(&csrc)
        .arg("-j16")
        .status()
        .expect("running make (hipcc --offload-arch=gfx950) for libvolta_hip.so");
    assert!(status.success(), "building libvolta_hip.so failed");
    println!("cargo:rustc-link-search=native={}", root.join("volta_amd").display());
    println!("cargo:rustc-link-lib=dylib=volta_hip");
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", root.join("include").join("volta_hip.h").display());
}
