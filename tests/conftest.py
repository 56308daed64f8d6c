"""Shared pytest setup: import paths, the `gpu` marker and common fixtures."""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "consumer-int8-kernels_amd"
for path in (REPO, PKG):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

LIB_PATH = PKG / "consumer_int8" / "libci8_amd.so"
HEADER_PATH = REPO / "include" / "consumer_int8_amd.h"
GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def ops():
    """The drop-in operator surface. On a GPU box a missing build is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    from consumer_int8 import ops as module

    return module


@pytest.fixture(scope="session")
def lib():
    """ctypes handle on the C ABI library."""
    from consumer_int8 import _abi

    return _abi.load()
