"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; everything else runs on
the CPU with the C oracle and the library's CPU-side entry points only.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


_TORCH_FIRST = []


@pytest.hookimpl(tryfirst=True)
def pytest_runtest_setup(item):
    """In a process that runs GPU tests, torch's HIP runtime initialises the GPU before the
    library's first call does (a torch tensor is made on cuda:0 before the first GPU test's
    fixtures run): torch's device initialisation after the library's has failed with
    "No HIP GPUs are available"."""
    if item.get_closest_marker("gpu") is None or _TORCH_FIRST:
        return
    _TORCH_FIRST.append(True)
    import torch
    if torch.cuda.device_count() > 0:
        torch.zeros(1, device="cuda:0")
