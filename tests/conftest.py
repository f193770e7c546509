"""Test configuration: the ``gpu`` marker and shared helpers.

CPU tests (``-m "not gpu"``) pin the oracle against the golden fixtures and check the C-ABI
library's exports and host-side argument validation.  GPU tests (``-m gpu``) compare the HIP
kernels, called through the C-ABI, with the oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def golden(name: str):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from mintext_amd import _lib

    _lib.lib()  # raises if the HIP library is missing: GPU tests never run without it
    return torch.device("cuda:0")


def rel_err(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b.ravel())
    return float(np.linalg.norm((a - b).ravel()) / (den if den > 0 else 1.0))


def tile_list_workspace_bytes(M: int, E: int) -> int:
    """The tile-list part of the grouped-GEMM workspace (mtx_gmm_workspace_size without the split
    tail): with it every tile runs whole, so any two kernels agree bit for bit."""
    up = lambda a, b: (a + b - 1) // b * b
    return up(up((48 + 2 * E + 1) * 4, 256) + (-(-M // 64) + E + 1) * 16, 256)
