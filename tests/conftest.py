"""Shared pytest setup: the `gpu` marker, import paths, and a reproducible generator per test.

GPU tests are marked `gpu` and skipped where no GPU is visible. The package under test is
gpu-spectral-stack_amd/python/spectral; the CPU oracle is oracle/ at the repository root.
"""

import sys
import zlib
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "gpu-spectral-stack_amd" / "python"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import torch  # noqa: E402  # before any library that links the HIP runtime


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built extension")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def rng(request) -> np.random.Generator:
    """Seeded from the test id, so every case draws the same numbers in any order
    (reference tests/conftest.py:20-24)."""
    return np.random.default_rng(zlib.crc32(request.node.nodeid.encode()))
