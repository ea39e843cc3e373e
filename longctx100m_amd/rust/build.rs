// build.rs of rust/longctx100m-model: compiles liblongctx100m_attn with hipcc for
// gfx950 (the flags of longctx100m_amd/build.py) and links the crate against it.
// Drop-in file for the reference crate; cargo is not part of this repository's
// toolchain, so it is not compiled here (tests/test_rust_binding.py checks its
// flags against longctx100m_amd/build.py).
use std::{env, fs, path::PathBuf, process::Command};

fn main() {
    let root = PathBuf::from(env::var("LONGCTX100M_AMD_ROOT")
        .expect("LONGCTX100M_AMD_ROOT: checkout of the MI355X library"));
    let csrc = root.join("longctx100m_amd/csrc");
    let include = root.join("include");
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".to_string());
    let mut objs = Vec::new();
    for entry in fs::read_dir(&csrc).expect("csrc") {
        let src = entry.unwrap().path();
        let ext = src.extension().and_then(|e| e.to_str()).unwrap_or("");
        println!("cargo:rerun-if-changed={}", src.display());
        if ext != "hip" && ext != "cpp" {
            continue;
        }
        let name = src.file_name().unwrap().to_string_lossy().into_owned();
        let obj = out.join(format!("{name}.o"));
        let mut cmd = Command::new(&hipcc);
        cmd.args(["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
                  "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .arg(format!("-I{}", include.display()));
        if name == "layer.hip" || name == "gemv.hip" {
            // the layer kernels round op by op like candle; the decode GEMVs fold the same ops
            cmd.arg("-ffp-contract=off");
        }
        let ok = cmd.arg("-c").arg(&src).arg("-o").arg(&obj).status().expect("run hipcc");
        assert!(ok.success(), "hipcc failed on {name}");
        objs.push(obj);
    }
    let lib = out.join("liblongctx100m_attn.so");
    let ok = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objs)
        .status()
        .expect("run hipcc (link)");
    assert!(ok.success(), "hipcc link failed");
    println!("cargo:rerun-if-changed={}", include.display());
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=longctx100m_attn");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
}
