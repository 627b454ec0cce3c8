"""Shared fixtures: the package (C ABI bindings), the CPU checker, and synthetic GGUFs.

Markers: tests marked `gpu` need an MI355X and call the HIP backend through the C ABI;
everything else runs on the CPU.
"""
from __future__ import annotations

import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP backend through the C ABI)")
    config.addinivalue_line("markers", "slow: full-size workloads (seconds of CPU checker time)")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("gguf")


_made = {}


@pytest.fixture(scope="session")
def gguf(pkg, model_dir):
    """gguf(preset) -> path of the preset's synthetic GGUF (written once per session)."""

    def make(preset: str) -> str:
        if preset not in _made:
            path = str(model_dir / f"{preset}.gguf")
            pkg.synth_write(preset, path)
            _made[preset] = path
        return _made[preset]

    return make


def n_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """Normwise relative error max|a-b| / max|b| (the 1e-3 activation bar)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = float(np.max(np.abs(b)))
    return float(np.max(np.abs(a - b))) / (den if den > 0 else 1.0)
