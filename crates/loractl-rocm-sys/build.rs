//! Builds libloractl_rocm.so with hipcc for gfx950 and links it.
//!
//! The HIP sources and the header are found through `LORACTL_ROCM_DIR` (a
//! checkout holding `loractl_amd/csrc/` and `include/`), by default the
//! repository this crate ships in (two levels up). `HIPCC` and `ROCM_PATH`
//! override the toolchain location. Only gfx950 code is generated; there is
//! no CUDA or other-architecture path.

use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

const SOURCES: [&str; 7] = [
    "lrq_quant.hip",
    "lrq_gemm.hip",
    "lrq_gemm_mid.hip",
    "lrq_skinny.hip",
    "lrq_lora.hip",
    "lrq_api.hip",
    "lrq_probe.hip",
];

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let root = env::var("LORACTL_ROCM_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join(".."));
    let csrc = root.join("loractl_amd").join("csrc");
    let include = root.join("include");
    let rocm = PathBuf::from(env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into()));
    let hipcc = env::var("HIPCC").map(PathBuf::from).unwrap_or_else(|_| rocm.join("bin").join("hipcc"));
    let out = PathBuf::from(env::var("OUT_DIR").expect("cargo sets OUT_DIR"));

    println!("cargo:rerun-if-env-changed=LORACTL_ROCM_DIR");
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed={}", include.join("loractl_rocm.h").display());
    for f in ["lrq_common.h", "lrq_kernels.h"] {
        println!("cargo:rerun-if-changed={}", csrc.join(f).display());
    }

    let mut objs = Vec::new();
    for src in SOURCES {
        let path = csrc.join(src);
        println!("cargo:rerun-if-changed={}", path.display());
        let obj = out.join(Path::new(src).with_extension("o"));
        let status = Command::new(&hipcc)
            .args(["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC"])
            // no packed-fp32 instructions: the kernels are written in scalar
            // and float2 code, and the compiler must not pair them
            .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .arg("-I")
            .arg(&include)
            .arg("-c")
            .arg(&path)
            .arg("-o")
            .arg(&obj)
            .status()
            .unwrap_or_else(|e| panic!("cannot run {}: {e}", hipcc.display()));
        assert!(status.success(), "hipcc failed on {}", path.display());
        objs.push(obj);
    }
    let lib = out.join("libloractl_rocm.so");
    let status = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objs)
        .status()
        .unwrap_or_else(|e| panic!("cannot run {}: {e}", hipcc.display()));
    assert!(status.success(), "hipcc failed to link {}", lib.display());

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=loractl_rocm");
    println!("cargo:rustc-link-search=native={}", rocm.join("lib").display());
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // found at run time next to the binary's rpath entries
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
}
