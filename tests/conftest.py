"""Shared test setup: import paths, the `gpu` marker and seeded input builders."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "comfyui-turing-utils_amd")
for path in (ROOT, PKG_DIR):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from comfyui_turing_utils_kernel import _lib

    dev = torch.device("cuda", 0)
    if not _lib.device_supported(dev):
        pytest.fail(f"device {torch.cuda.get_device_name(0)} is not gfx950")
    return dev
