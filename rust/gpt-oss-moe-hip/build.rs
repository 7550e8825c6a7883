//! Builds libgossmx.so for gfx950 with hipcc, straight from the C++/HIP
//! sources (no cmake, no Python): the same sources and flags as
//! gpt-oss-rs_amd/build.py. The HIP sources are compiled for the device and
//! the host; the store and the dense path are host-only C++.

use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

const HIP_SOURCES: [&str; 2] = ["gossmx_kernels.hip", "gossmx_api.hip"];
const HOST_SOURCES: [&str; 2] = ["gossmx_store.cpp", "gossmx_dense.cpp"];

fn hipcc() -> PathBuf {
    if let Ok(path) = env::var("HIPCC") {
        return PathBuf::from(path);
    }
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    Path::new(&rocm).join("bin").join("hipcc")
}

fn run(cmd: &mut Command, what: &str) {
    let status = cmd.status().unwrap_or_else(|error| panic!("{what}: cannot run hipcc: {error}"));
    assert!(status.success(), "{what} failed with {status}");
}

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let root = env::var("GOSSMX_ROOT")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join(".."));
    let csrc = root.join("gpt-oss-rs_amd").join("csrc");
    let include = root.join("include");
    let out = PathBuf::from(env::var("OUT_DIR").expect("OUT_DIR"));
    let hipcc = hipcc();
    let rocm_include = env::var("ROCM_PATH").map(|p| format!("{p}/include")).unwrap_or("/opt/rocm/include".into());

    // -ffp-contract=off keeps every multiply and add of the reference's float
    // chains separate; packed f32 instructions stay off in device code.
    let device_flags = [
        "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ];
    let host_flags = ["-x", "c++", "-D__HIP_PLATFORM_AMD__", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off"];

    let mut objects = Vec::new();
    for src in HIP_SOURCES {
        let obj = out.join(format!("{src}.o"));
        run(
            Command::new(&hipcc).args(device_flags).arg("-I").arg(&include).arg("-c").arg(csrc.join(src)).arg("-o").arg(&obj),
            src,
        );
        objects.push(obj);
    }
    for src in HOST_SOURCES {
        let obj = out.join(format!("{src}.o"));
        run(
            Command::new(&hipcc)
                .args(host_flags)
                .arg(format!("-I{rocm_include}"))
                .arg("-I")
                .arg(&include)
                .arg("-c")
                .arg(csrc.join(src))
                .arg("-o")
                .arg(&obj),
            src,
        );
        objects.push(obj);
    }
    let lib = out.join("libgossmx.so");
    run(
        Command::new(&hipcc).args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"]).arg(&lib).args(&objects),
        "link libgossmx.so",
    );

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=gossmx");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", include.join("gossmx.h").display());
    println!("cargo:rerun-if-env-changed=GOSSMX_ROOT");
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
