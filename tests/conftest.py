"""Shared test set-up.

* ``gpu`` marks tests that need the MI355X (``pytest -m gpu``); everything else
  runs on a CPU-only machine (``pytest -m "not gpu"``).
* The repository root (for ``oracle``) and ``oko-xpu-kernels_amd`` (for the
  ``xpu_kernels`` package) go on ``sys.path``.
"""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "oko-xpu-kernels_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built library")


@pytest.fixture(scope="session")
def dev():
    """The GPU device, with the library loaded -- or a hard failure: a GPU test
    must never pass on a fallback."""
    import torch
    from xpu_kernels import int8
    from xpu_kernels.int8 import _lib as L
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    assert int8.available(), f"libxpuint8 did not load: {L._ERR}"
    return torch.device("cuda", 0)


def seeded(seed):
    return np.random.default_rng(seed)
