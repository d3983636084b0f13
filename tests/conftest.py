"""pytest configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` runs the CPU suite (oracle pinning, host logic, C-ABI symbol
checks); ``-m gpu`` runs the parity tests on an MI355X through the C-ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "log-linear-attention_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(autouse=True)
def _skip_gpu_without_device(request):
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("no GPU visible")
