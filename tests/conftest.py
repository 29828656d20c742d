"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the CPU suite (oracle pins, host-side API behaviour,
C-ABI exports).  ``-m gpu`` runs the parity tests of the HIP kernels against
the CPU oracle; they need a ROCm GPU and the built library.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "smooth-attn_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
