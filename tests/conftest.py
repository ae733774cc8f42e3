"""Shared test setup: import paths, the `gpu` marker, and skipping GPU tests where no GPU is visible.

`python -m pytest tests -m "not gpu"` runs the CPU suite (oracle pinning, host logic, library loading);
`python -m pytest tests -m gpu` runs the parity tests of the HIP kernels against the oracle on an MI355X.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "small-inference_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
