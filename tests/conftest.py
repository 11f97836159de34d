"""pytest configuration: import paths and the ``gpu`` marker.

CPU tests (``-m "not gpu"``) check the oracle against closed forms, library
routines and brute force, the host-side logic, and that the C-ABI library
loads and exports every declared symbol.  GPU tests (``-m gpu``) are the
parity tests proper: they run the HIP kernels through the C ABI and compare
with the oracle on the same seeded inputs.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "dimmer-kv_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
