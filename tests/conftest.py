"""Test configuration: the `gpu` marker, import paths, shared fixtures.

`-m "not gpu"` runs on any host (oracle against golden vectors and closed forms, host logic, the
C-ABI library's exports). `-m gpu` needs a ROCm GPU and calls the HIP kernels through the C ABI.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "blackhole-harness_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU on this host")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
