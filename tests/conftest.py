"""Shared fixtures: the HIP library binding, the CPU oracle, input generators.

Tests marked `gpu` need an MI355X; everything else runs on the CPU (the C-ABI
library is loaded there too, but only entry points that fail before touching
the device are called).
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PKG_DIR = REPO / "ternary-bonsai-inference_amd"


def _load(name: str, path: Path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, path, submodule_search_locations=[str(path.parent)] if path.name == "__init__.py" else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_bonsai():
    return _load("bonsai_amd", PKG_DIR / "__init__.py")


def load_synth():
    return _load("bonsai_amd_synth", PKG_DIR / "synth.py")


def load_oracle():
    return _load("bonsai_oracle", REPO / "oracle" / "oracle.py")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def bh():
    return load_bonsai()


@pytest.fixture(scope="session")
def synth():
    return load_synth()


@pytest.fixture(scope="session")
def oracle():
    return load_oracle()


@pytest.fixture(scope="session")
def dev():
    """The GPU; fails (does not skip) when a gpu-marked test has none."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible GPU")
    return torch.device("cuda:0")


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max(max|ref|, max|got|) -- the reference's per-tensor
    metric (src/bin/bonsai-actcmp.rs:53-62).  NaN positions must match."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), "NaN positions differ"
    g, r = got[~gn], ref[~rn]
    if g.size == 0:
        return 0.0
    # infinities must match exactly
    gi, ri = np.isinf(g), np.isinf(r)
    assert np.array_equal(gi, ri) and np.array_equal(g[gi], r[ri]), "inf entries differ"
    g, r = g[~gi].astype(np.float64), r[~ri].astype(np.float64)
    if g.size == 0:
        return 0.0
    den = max(np.abs(r).max(), np.abs(g).max(), 1e-30)
    return float(np.abs(g - r).max() / den)


def bits_equal(got, ref) -> bool:
    a = np.ascontiguousarray(got, dtype=np.float32).view(np.uint32)
    b = np.ascontiguousarray(ref, dtype=np.float32).view(np.uint32)
    return a.shape == b.shape and bool(np.array_equal(a, b))
