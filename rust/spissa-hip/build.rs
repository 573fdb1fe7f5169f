//! Builds libspissa_hip.so from the HIP sources of this repository with hipcc,
//! exactly as spissa_amd/build.py does: every `*.hip` file of spissa_amd/csrc
//! (a directory listing, so a new kernel file needs no edit here), the same
//! flags for every file (COMMON), the same per-file additions (EXTRA) and the
//! same link line. tests/test_integration_recipe.py compares these constants
//! with build.py.
//!
//! The sources are found through SPISSA_HIP_SRC (the spissa_amd directory), or
//! else at ../../spissa_amd from this crate's real location (a symlink such as
//! crates/spissa-hip in the Spissa workspace resolves to rust/spissa-hip here).
//! ROCM_PATH (default /opt/rocm) locates hipcc and libamdhip64.
use std::{env, fs, path::PathBuf, process::Command};

/// Flags of every hipcc compile (spissa_amd/build.py COMMON, without its -I).
const COMMON: &[&str] = &[
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Wno-unused-command-line-argument", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
];
/// Per-source additions (spissa_amd/build.py EXTRA): prefill.hip keeps MFMA
/// results in VGPRs.
const EXTRA: &[(&str, &[&str])] = &[
    ("prefill.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
];
/// The link line (spissa_amd/build.py build()): flags, objects, libraries.
const LINK: &[&str] = &["--offload-arch=gfx950", "-shared", "-fPIC"];
const LINK_LIBS: &[&str] = &["-lpthread"];

fn source_root() -> PathBuf {
    if let Ok(dir) = env::var("SPISSA_HIP_SRC") {
        return PathBuf::from(dir);
    }
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let real = fs::canonicalize(&manifest).unwrap_or(manifest);
    real.join("../../spissa_amd")
}

fn main() {
    let root = source_root();
    let out = PathBuf::from(env::var("OUT_DIR").expect("OUT_DIR"));
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    let hipcc = format!("{rocm}/bin/hipcc");
    let include = format!("-I{}", root.join("../include").display());
    // every csrc/*.hip, in name order (build.py: sorted(CSRC.glob("*.hip")))
    let mut srcs: Vec<PathBuf> = fs::read_dir(root.join("csrc"))
        .unwrap_or_else(|e| panic!("cannot list {}: {e}", root.join("csrc").display()))
        .map(|e| e.expect("csrc entry").path())
        .filter(|p| p.extension().map_or(false, |x| x == "hip"))
        .collect();
    srcs.sort();
    assert!(!srcs.is_empty(), "no HIP sources under {}", root.join("csrc").display());
    let mut objs = Vec::new();
    for src in &srcs {
        let name = src.file_name().unwrap().to_str().unwrap();
        let extra: &[&str] = EXTRA.iter().find(|(n, _)| *n == name).map_or(&[], |(_, f)| f);
        let obj = out.join(src.with_extension("o").file_name().unwrap());
        let st = Command::new(&hipcc)
            .args(COMMON)
            .args(extra)
            .arg(&include)
            .arg("-c")
            .arg(src)
            .arg("-o")
            .arg(&obj)
            .status()
            .expect("hipcc");
        assert!(st.success(), "hipcc failed on {}", src.display());
        println!("cargo:rerun-if-changed={}", src.display());
        objs.push(obj);
    }
    println!("cargo:rerun-if-changed={}", root.join("csrc").display());
    println!("cargo:rerun-if-changed={}", root.join("../include/spissa_hip.h").display());
    println!("cargo:rerun-if-env-changed=SPISSA_HIP_SRC");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    let lib = out.join("libspissa_hip.so");
    let st = Command::new(&hipcc)
        .args(LINK)
        .arg("-o")
        .arg(&lib)
        .args(&objs)
        .args(LINK_LIBS)
        .status()
        .expect("hipcc link");
    assert!(st.success(), "link of {} failed", lib.display());
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=spissa_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
