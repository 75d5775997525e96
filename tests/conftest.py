"""Test configuration: puts the repo root (for ``oracle``) and the package
directory (for ``warp_route``) on sys.path and registers the ``gpu`` marker.

CPU tests (``-m "not gpu"``) cover the oracle, the layout, host-side argument
validation and the C-ABI library's exports.  GPU tests (``-m gpu``) are the
parity tests proper and run the HIP kernels through the C-ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "warp-route_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch.device("cuda:0")
