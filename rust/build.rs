// build.rs -- compile the HIP kernels for gfx950 and link them.
//
// These are lines to add to the reference's existing build script: call
// build_hip() from its fn main() (this file has no main of its own).
// Layout it expects, relative to the crate root (where build.rs lives):
//   hip/csrc/     the csrc/ directory of this repository
//   include/      the include/ directory of this repository
// csrc/common.hpp includes "../../include/bonsai_hip.h", which from
// hip/csrc/ resolves to include/ at the crate root.
fn build_hip() {
    let out = std::path::PathBuf::from(std::env::var("OUT_DIR").unwrap());
    let src = "hip/csrc"; // the csrc/ directory of this repository, vendored
    assert!(std::path::Path::new("include/bonsai_hip.h").exists(),
            "vendor this repository's include/ at the crate root (hip/csrc includes ../../include)");
    let mut objs = Vec::new();
    for f in std::fs::read_dir(src).unwrap() {
        let p = f.unwrap().path();
        let ext = p.extension().and_then(|e| e.to_str()).unwrap_or("");
        if ext != "hip" && ext != "cpp" { continue; }
        let o = out.join(p.file_name().unwrap()).with_extension("o");
        let mut cmd = std::process::Command::new("/opt/rocm/bin/hipcc");
        if ext == "hip" { cmd.arg("--offload-arch=gfx950"); }
        cmd.args(["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
                  "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-c"])
           .arg(&p).arg("-o").arg(&o);
        assert!(cmd.status().unwrap().success(), "hipcc failed on {:?}", p);
        objs.push(o);
    }
    let lib = out.join("libbonsai_hip.so");
    let st = std::process::Command::new("/opt/rocm/bin/hipcc")
        .args(["--offload-arch=gfx950", "-shared", "-fPIC"]).args(&objs)
        .arg("-o").arg(&lib).status().unwrap();
    assert!(st.success());
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=bonsai_hip");
    println!("cargo:rustc-link-search=native=/opt/rocm/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-changed={}", src);
}
