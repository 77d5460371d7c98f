"""Build step of the bonsai HIP library: hipcc for gfx950, in-tree output.

Compiles every source under csrc/ to an object in _build/ and links
lib/libbonsai_hip.so next to this file.  Always recompiles (the driver's
"does it build" check relies on that).  Also builds the CPU oracle under
oracle/ (the test checker) with its Makefile.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libbonsai_hip.so"
ORACLE_DIR = REPO / "oracle"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: no FMA contraction, so every f32 product and sum rounds
#   as in the reference's Rust (which never contracts).
# -packed-fp32-ops off: keep the compiler from emitting packed FP32 math.
COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        # host-only translation units: no device code object needed
        cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build_library(jobs: int | None = None) -> Path:
    """Compile and link lib/libbonsai_hip.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = jobs or min(8, len(sources))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


CPP_TEST_SRC = REPO / "tests" / "cpp" / "test_kernels.cpp"
CPP_TEST_BIN = REPO / "tests" / "cpp" / "test_kernels"


def build_cpp_tests() -> Path:
    """Host-only C++ program restating the reference's unit tests against the
    C++ interface mirror (host/bonsai_kernels.hpp), linked to the library."""
    cmd = [HIPCC, "-O2", "-std=c++17", str(CPP_TEST_SRC), "-o", str(CPP_TEST_BIN),
           f"-L{LIB.parent}", "-lbonsai_hip", f"-Wl,-rpath,{LIB.parent}",
           "-Wl,-rpath,$ORIGIN/../../ternary-bonsai-inference_amd/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"C++ mirror tests failed to build:\n{res.stderr}")
    return CPP_TEST_BIN


def build_oracle() -> Path:
    """Build oracle/liboracle.so (test infrastructure) with its Makefile."""
    res = subprocess.run(["make", "-B", "-C", str(ORACLE_DIR)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return ORACLE_DIR / "liboracle.so"


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    print(build_library())
    print(build_cpp_tests())
    print(build_oracle())
