"""Shared test setup: import paths, the gpu marker, and cached model weights."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "oracle")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def clf_weights():
    from ironicl_amd import synthetic

    return synthetic.random_weights("classifier")


@pytest.fixture(scope="session")
def reg_weights():
    from ironicl_amd import synthetic

    return synthetic.random_weights("regressor")


def lcg_values(count: int, state: int = 1, scale: float = 12.0) -> np.ndarray:
    """The reference's LCG test data: state = state * 1664525 + 1013904223
    (mod 2^32), value = (state / u32::MAX - 0.5) * 12 (src/kernels/reference.rs:1862-1872)."""
    out = np.empty(count, np.float32)
    for i in range(count):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((np.float32(state) / np.float32(4294967295.0) - np.float32(0.5)) * np.float32(scale))
    return out, state
