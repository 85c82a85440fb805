"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; everything else runs on
the CPU with the C oracle and the library's CPU-side entry points only.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
