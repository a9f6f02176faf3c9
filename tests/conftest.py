"""Shared pytest configuration: the `gpu` marker and GPU/library fixtures.

CPU tests (`-m "not gpu"`) cover the oracle against the golden vectors, the host-side logic of
the C ABI and that the library exports every declared symbol. GPU tests (`-m gpu`) are the
parity tests proper: they call the HIP kernels through the C ABI and compare with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library (calls kernels)")


@pytest.fixture(scope="session")
def dev():
    """The GPU device; fails loudly (never skips) when the HIP runtime or library is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU test selected but no GPU is visible"
    from bitgpu_amd._lib import lib
    lib()  # raises if the HIP library was not built
    return "cuda"


def rel_err(got, want):
    import numpy as np
    return float(np.abs(got - want).max() / max(float(np.abs(want).max()), 1e-30))


def cosine(a, b):
    import numpy as np
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
