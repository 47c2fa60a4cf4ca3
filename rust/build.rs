//! Build script of the MI355X device layer.
//!
//! Replaces the reference's build.rs (build.rs:1-60), which compiles
//! src/cuda/nn_math.cu to PTX with nvcc and embeds it: here the device code is
//! the prebuilt HIP library `libsoklyn_hip.so` (gfx950 code objects, C ABI of
//! include/soklyn_hip.h), linked like any shared library.  SOKLYN_HIP_DIR names
//! a directory that holds it; without it the library is built from
//! soklyn_amd/csrc with the repository's own build step (hipcc).
use std::path::PathBuf;
use std::process::Command;

fn main() {
    println!("cargo:rerun-if-env-changed=SOKLYN_HIP_DIR");
    let manifest = PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let repo = manifest.join("..");
    let lib_dir = match std::env::var("SOKLYN_HIP_DIR") {
        Ok(dir) => PathBuf::from(dir),
        Err(_) => {
            let status = Command::new("python3")
                .args(["-m", "soklyn_amd.build"])
                .current_dir(&repo)
                .status()
                .expect("python3 is needed to build libsoklyn_hip.so (or set SOKLYN_HIP_DIR)");
            assert!(status.success(), "building libsoklyn_hip.so failed: {status}");
            repo.join("soklyn_amd")
        }
    };
    for src in ["abi.hip", "gemm.hip", "elementwise.hip", "gemm.h", "gemm_dma.h", "device_math.h"] {
        println!("cargo:rerun-if-changed={}", repo.join("soklyn_amd/csrc").join(src).display());
    }
    println!("cargo:rerun-if-changed={}", repo.join("include/soklyn_hip.h").display());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=soklyn_hip");
    // the library finds libamdhip64 through its own runpath; the binary finds the library here
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
}
