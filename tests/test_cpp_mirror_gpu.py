"""Runs tests/cpp/test_kernels: the reference's own unit tests restated in C++
against the interface mirror (host/bonsai_kernels.hpp) on the GPU."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "test_kernels"


@pytest.mark.gpu
def test_reference_unit_tests_through_cpp_mirror(dev):
    assert BIN.exists(), "tests/cpp/test_kernels not built: run __graft_entry__.build()"
    res = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.count("PASS ") == 14 and "FAIL" not in res.stdout


def test_cpp_mirror_program_is_built():
    assert BIN.exists(), "tests/cpp/test_kernels not built: run __graft_entry__.build()"
