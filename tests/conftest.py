"""Shared test setup: the ``gpu`` marker, the package fixture and bf16 helpers.

GPU tests are marked ``gpu`` and call the HIP kernels through the C ABI; everything else runs on
the CPU (oracle pinning, host-side logic, library loading and exported symbols).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1.6e-2, 1e-2     # bf16 tolerance for the floating-point ops


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU and the built HIP kernel library")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def mas():
    """The package, imported from mini-agent-serve_amd/."""
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda:0")


def bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a bf16 tensor (copied to the host)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    """bf16 tensor (CPU) holding the given uint16 bit patterns."""
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def fp8_codes(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()
