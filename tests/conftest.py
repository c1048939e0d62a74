"""Shared test configuration.

* `-m gpu` tests need a gfx950 GPU and the built libsiliconfer_hip.so; they run
  on the GPU box. Without any GPU they skip; with a GPU but no library (or a
  non-gfx950 device) they FAIL, since the product has no fallback.
* everything else runs on the CPU: the oracle against golden vectors and
  closed forms, the host-side API, and the C-ABI's exports / argument checks.
"""

from __future__ import annotations

import glob
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


def golden_cases(prefix: str = ""):
    return sorted(os.path.basename(p)[:-4]
                  for p in glob.glob(os.path.join(GOLDEN_DIR, f"{prefix}*.npz")))


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="session")
def hip():
    """The loaded HIP library for GPU tests (skips only when no GPU exists)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from siliconfer_amd import _lib

    lib = _lib.load()  # raises if not built: a GPU box without the library is a failure
    assert lib.sf_device_arch_ok(torch.cuda.current_device()) == 1, "device is not gfx950"
    return lib


@pytest.fixture
def dev(hip):
    import torch

    return torch.device("cuda", torch.cuda.current_device())
