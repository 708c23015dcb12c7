//! Builds libiris_hip.so from its HIP sources with hipcc for gfx950 and links
//! it dynamically (the HIP runtime, amdhip64, comes with it), or links a
//! library built beforehand.
//!
//! - `IRIS_HIP_LIB_DIR`: a directory holding a built libiris_hip.so; nothing
//!   is compiled.
//! - `IRIS_HIP_SRC`: the directory of the library's `.hip` sources (default:
//!   the package's `csrc`, ../../iris_amd/csrc from this crate).
//! - `ROCM_PATH`: the ROCm installation (default /opt/rocm).

use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

fn run(command: &mut Command) {
    let status = command
        .status()
        .unwrap_or_else(|error| panic!("failed to start {command:?}: {error}"));
    assert!(status.success(), "{command:?} failed");
}

fn main() {
    println!("cargo:rerun-if-changed=build.rs");
    println!("cargo:rerun-if-env-changed=IRIS_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=IRIS_HIP_SRC");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());

    let lib_dir = match env::var_os("IRIS_HIP_LIB_DIR") {
        Some(dir) => PathBuf::from(dir),
        None => {
            let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
            let src = env::var_os("IRIS_HIP_SRC")
                .map(PathBuf::from)
                .unwrap_or_else(|| manifest.join("../../iris_amd/csrc"));
            let out = PathBuf::from(env::var("OUT_DIR").unwrap());
            build_library(&rocm, &src, &out);
            out
        }
    };
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=iris_hip");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // Found at run time beside the binary or through the build's path.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
}

/// One object per `.hip` file (packed FP32 VALU forms off), linked into
/// libiris_hip.so.
fn build_library(rocm: &str, src: &Path, out: &Path) {
    let hipcc = format!("{rocm}/bin/hipcc");
    let mut objects = Vec::new();
    let mut sources: Vec<PathBuf> = std::fs::read_dir(src)
        .unwrap_or_else(|error| panic!("cannot read {}: {error}", src.display()))
        .filter_map(|entry| entry.ok().map(|e| e.path()))
        .filter(|path| path.extension().is_some_and(|ext| ext == "hip"))
        .collect();
    sources.sort();
    for source in &sources {
        println!("cargo:rerun-if-changed={}", source.display());
        let object = out.join(source.file_name().unwrap()).with_extension("o");
        run(Command::new(&hipcc)
            .args(["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950"])
            .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .arg("-c")
            .arg(source)
            .arg("-o")
            .arg(&object));
        objects.push(object);
    }
    for header in ["detnum_dev.h", "q8_internal.h", "q8_epilogue.h", "layer_kernels.h", "runtime_internal.h"] {
        println!("cargo:rerun-if-changed={}", src.join(header).display());
    }
    run(Command::new(&hipcc)
        .args(["-shared", "-fPIC", "--offload-arch=gfx950"])
        .args(&objects)
        .arg("-o")
        .arg(out.join("libiris_hip.so")));
}
