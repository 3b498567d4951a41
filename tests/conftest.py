"""pytest configuration: the ``gpu`` marker and import paths.

Tests marked ``gpu`` need a ROCm device and the built HIP library; they call
the product through its C-ABI.  Everything else runs on a CPU-only host.
"""
from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950) and the HIP library")
