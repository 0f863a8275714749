"""Shared test setup: import paths, the `gpu` marker, and common helpers.

`-m "not gpu"` tests run anywhere (host layer, oracle vs closed forms,
library loading); `-m gpu` tests need an MI355X and call the device library
through its C ABI / the compiled executor.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "lets-build-a-runtime_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built device library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def normwise_rel(y, ref) -> float:
    """max|y - ref| / max|ref| — the parity metric (≤ 1e-3 for fp32 paths)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.abs(ref).max()) if ref.size else 0.0
    return float(np.abs(y - ref).max()) / den if den > 0 else float(np.abs(y - ref).max())


@pytest.fixture(scope="session")
def hip_lib():
    """The device library, initialised on device 0 (gpu tests only)."""
    from runtime.executor.hip_lib import load_library
    return load_library(0)
