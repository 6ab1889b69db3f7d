"""Shared pytest configuration.

Markers:
  gpu -- needs a real MI355X (gfx950) GPU; CPU-only runs deselect these with
         ``-m "not gpu"``.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an MI355X GPU (HIP)")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test needs a GPU; deselect with -m 'not gpu'")
    return torch.device("cuda:0")
