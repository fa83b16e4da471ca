//! Builds libflour_hip.so for gfx950 from the HIP sources of this repository and links it.
//!
//! The sources live in `flour_amd/csrc` two directories up; `python3 -m flour_amd.build`
//! compiles every `.hip` / `.cpp` file there with `hipcc --offload-arch=gfx950` (packed FP32
//! instructions disabled) and links `flour_amd/libflour_hip.so`. Set `FLOUR_AMD_ROOT` to use a
//! checkout elsewhere, and `FLOUR_HIP_ARCH` to build for another target.
use std::path::PathBuf;
use std::process::Command;

fn main() {
    let root = match std::env::var("FLOUR_AMD_ROOT") {
        Ok(p) => PathBuf::from(p),
        Err(_) => PathBuf::from(env!("CARGO_MANIFEST_DIR")).join("../.."),
    };
    let status = Command::new("python3")
        .args(["-m", "flour_amd.build"])
        .current_dir(&root)
        .status()
        .expect("running python3 -m flour_amd.build (needs hipcc from ROCm)");
    assert!(status.success(), "building libflour_hip.so failed");
    let lib_dir = root.join("flour_amd");
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=flour_hip");
    // the shared library is found at run time next to the build, as hipcc linked it
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-changed={}", root.join("flour_amd/csrc").display());
    println!("cargo:rerun-if-changed={}", root.join("include").display());
    println!("cargo:rerun-if-env-changed=FLOUR_AMD_ROOT");
    println!("cargo:rerun-if-env-changed=FLOUR_HIP_ARCH");
}
