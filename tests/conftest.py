"""Shared test setup: import paths, the `gpu` marker, small helpers."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "rina-1bit-kv_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def kv_like(rng, shape, outliers=True):
    """N(0,1) values, optionally times log-normal(sigma=1) per-channel scales (last axis)."""
    x = rng.standard_normal(shape).astype(np.float32)
    if outliers:
        x *= np.exp(rng.standard_normal(shape[-1])).astype(np.float32)
    return x
