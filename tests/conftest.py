"""Shared pytest configuration.

Markers:
  gpu — needs a HIP device and the built libnacho_hip.so; run on the MI355X box with
        `pytest -m gpu`.  Everything unmarked runs on the CPU.
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and libnacho_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device tests run on; fails (never skips) when it is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    import nacho_amd._lib as lib

    lib.load()  # raises if the library is not built: no silent fallback
    return torch.device("cuda:0")
