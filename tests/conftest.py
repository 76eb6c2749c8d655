"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (gfx950) and the built HIP library; all
other tests run on the CPU (oracle checks, host-side validation, ABI exports).
"""
import os
import sys

import pytest

# PyTorch-ROCm ships its own HIP runtime.  Loading torch before anything that
# links the system libamdhip64 (bten, libbnhip) keeps one runtime per process.
import torch  # noqa: F401

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "baranet-bdml_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
