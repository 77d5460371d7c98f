"""CPU check of the closed form for runs of identical sequential f32 additions
(csrc/seqsum.hpp) that the fused gather + RMSNorm uses to reproduce the
reference's sequential sum of squares (src/kernels.rs:65-68) bit for bit.

tests/cpp/test_seqsum.cpp compares it with the plain addition loop on random
runs (all binade offsets, ties, sums just below a binade boundary, n up to
5000) and on whole ternary rows of 40 f16-scaled blocks."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "cpp" / "test_seqsum.cpp"


@pytest.mark.parametrize("rcp_ulp", [0, -1, 1])
def test_repeat_add_matches_sequential_loop(tmp_path, rcp_ulp):
    """rcp_ulp moves the reciprocal of the step count one ulp down or up:
    the GPU's approximate reciprocal may err either way by that much."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = tmp_path / "test_seqsum"
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", f"-DRCP_ULP={rcp_ulp}",
                    str(SRC), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert " 0 mismatches" in res.stdout
