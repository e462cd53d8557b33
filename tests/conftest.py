"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` tests run anywhere (oracle, host logic, library exports);
``-m gpu`` tests need a gfx950 device and call the HIP kernels through the C ABI.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "sglang-lite_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def gpu():
    """The device the GPU tests run on; fails loudly when the library cannot run there."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    import sglang_lite_amd

    info = sglang_lite_amd.probe()
    assert info["ok"], f"sglang_lite_amd probe failed on the GPU: {info}"
    return torch.device("cuda:0")
