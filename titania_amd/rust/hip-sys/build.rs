//! Compiles every `.hip` source of the hip device for gfx950 (the flags of
//! titania_amd/build.py) and links the shared library beside the crate's
//! output.
use std::{env, path::PathBuf, process::Command};

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let src = manifest.join("../../csrc");
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let mut objs = Vec::new();
    for entry in std::fs::read_dir(&src).unwrap() {
        let path = entry.unwrap().path();
        let ext = path.extension().and_then(|e| e.to_str());
        if ext == Some("h") {
            println!("cargo:rerun-if-changed={}", path.display());
        }
        if ext != Some("hip") {
            continue;
        }
        let obj = out.join(path.file_stem().unwrap()).with_extension("o");
        let ok = Command::new(&hipcc)
            .args(["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-fvisibility=hidden",
                   "-fvisibility-inlines-hidden", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                   "-c"])
            .arg(&path)
            .arg("-o")
            .arg(&obj)
            .status()
            .expect("hipcc not found")
            .success();
        assert!(ok, "hipcc failed on {}", path.display());
        objs.push(obj);
        println!("cargo:rerun-if-changed={}", path.display());
    }
    let lib = out.join("libtitania_hip.so");
    let ok = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC"])
        .args(&objs)
        .arg("-o")
        .arg(&lib)
        .status()
        .expect("hipcc not found")
        .success();
    assert!(ok, "linking libtitania_hip.so failed");
    println!("cargo:rerun-if-changed={}", manifest.join("../../../include/titania_hip.h").display());
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=titania_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
}
