//! Compiles the backend's HIP and C++ sources with hipcc for gfx950 into liborca_hip.so in
//! OUT_DIR and links the crate against it (the same flags as orcaml_amd/build.py):
//! -ffp-contract=off keeps the reference's separate f32 multiply and add in elementwise and
//! optimizer arithmetic, and packed-FP32 instructions are switched off.
//!
//! Environment: ORCAML_AMD_DIR (the `orcaml_amd` package directory, default ../orcaml_amd),
//! HIPCC (default /opt/rocm/bin/hipcc).
use std::env;
use std::fs;
use std::path::{Path, PathBuf};
use std::process::Command;

const SOURCES: [&str; 9] = [
    "runtime_host.cpp",
    "storage.cpp",
    "runtime.hip",
    "ops.hip",
    "gemm.hip",
    "fused.hip",
    "head.hip",
    "mlp.hip",
    "ewprog.hip",
];

fn run(cmd: &mut Command) {
    let status = cmd.status().unwrap_or_else(|e| panic!("failed to start {:?}: {}", cmd, e));
    if !status.success() {
        panic!("{:?} failed with {}", cmd, status);
    }
}

fn main() {
    let pkg = PathBuf::from(env::var("ORCAML_AMD_DIR").unwrap_or_else(|_| "../orcaml_amd".to_string()));
    let csrc = pkg.join("csrc");
    let out = PathBuf::from(env::var("OUT_DIR").expect("OUT_DIR"));
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".to_string());

    // ewprog.hip hands the functor header's text to hipRTC: embed it as a raw string literal.
    let ops = fs::read_to_string(csrc.join("ew_ops.hpp")).expect("ew_ops.hpp");
    assert!(!ops.contains(")EWOPS\""), "ew_ops.hpp contains the raw-string delimiter");
    fs::write(out.join("ew_ops_text.inc"), format!("R\"EWOPS({})EWOPS\"\n", ops)).expect("ew_ops_text.inc");

    let mut objs = Vec::new();
    for src in SOURCES.iter() {
        let path = csrc.join(src);
        println!("cargo:rerun-if-changed={}", path.display());
        let obj = out.join(format!("{}.o", src.replace('.', "_")));
        run(Command::new(&hipcc)
            .args(["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off"])
            .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .arg("-I")
            .arg(&out)
            .arg("-c")
            .arg(&path)
            .arg("-o")
            .arg(&obj));
        objs.push(obj);
    }
    for hdr in ["runtime.hpp", "ew_ops.hpp", "ce_row.hpp"].iter() {
        println!("cargo:rerun-if-changed={}", csrc.join(hdr).display());
    }
    println!("cargo:rerun-if-changed={}", Path::new(&pkg).join("../include/orca_hip.h").display());
    let lib = out.join("liborca_hip.so");
    run(Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objs)
        .arg("-ldl"));
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=orca_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
}
