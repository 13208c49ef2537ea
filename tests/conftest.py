"""Test setup: import paths, the ``gpu`` marker, shared helpers.

GPU tests are the parity tests proper: they call the HIP kernels through the C ABI and compare with
the CPU oracle under ``oracle/``.  Without a visible GPU they are skipped; with one, a missing
library is an error (ptb_amd has no fallback).
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "pytorchsim-triton-backend_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libptb_amd.so")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
