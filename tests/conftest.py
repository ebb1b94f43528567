"""pytest configuration: the ``gpu`` marker and shared helpers.

``-m "not gpu"`` runs everywhere (oracle pinning, host logic, C-ABI loading
and argument errors); ``-m gpu`` needs a ROCm device and the in-tree
``avelang_amd/libgdn.so``.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


def has_rocm() -> bool:
    """ROCm device present (python/avelang/testing.py:21-26 convention)."""
    import torch

    return torch.cuda.is_available() and getattr(torch.version, "hip", None) is not None


@pytest.fixture(scope="session")
def rocm_device():
    if not has_rocm():
        pytest.skip("Requires ROCm/HIP with an AMD GPU.")
    import torch

    return torch.device("cuda:0")
