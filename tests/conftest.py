"""pytest configuration: the `gpu` marker and shared fixtures.

  python -m pytest tests -m "not gpu"   # CPU: oracle pinning, dispatch contract, C ABI
  python -m pytest tests -m gpu         # MI355X: HIP kernels vs the oracle
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    return torch.device("cuda", 0)
