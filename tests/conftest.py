"""Shared pytest setup.

* puts the package directory (mhc-triton_amd/) and the repo root on sys.path so
  ``import mhc`` and ``import oracle`` work from a checkout;
* registers the ``gpu`` marker: ``-m gpu`` selects the parity tests that run the
  HIP library on a ROCm GPU, ``-m "not gpu"`` the CPU suite (oracle pins, host
  logic, ABI exports).  GPU tests skip when no GPU is visible.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "mhc-triton_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for it in gpu_items:
        it.add_marker(skip)

