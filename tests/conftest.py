"""Test setup: import paths, the ``gpu`` marker, output poisoning.

GPU tests are the parity tests proper: they call the HIP kernels through the C ABI and compare with
the CPU oracle under ``oracle/``.  Without a visible GPU they are skipped; with one, a missing
library is an error (ptb_amd has no fallback).

Every GPU tensor a ``gpu`` test allocates with ``torch.empty`` / ``torch.empty_like`` -- the outputs
and workspaces ``ptb_amd`` allocates for a call as well as the ones a test passes in -- is filled
with a poison pattern first (NaN for floating dtypes, the e4m3 NaN byte for fp8, 0xA5 bytes for
integers), so an element a kernel fails to write cannot pass on bytes an earlier launch left in the
caching allocator.  The reference's device does the same for its outputs (runtime/spike.py:310-334
checks conflicting and missing writes).
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


def poison_(t):
    """Fill a fresh GPU tensor with the poison pattern of its dtype (in place; returns it)."""
    import torch

    if t.device.type != "cuda" or t.numel() == 0 or t.dtype == torch.bool:
        return t
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        t.view(torch.uint8).fill_(0x7F)                # NaN in both fp8 formats
    elif t.is_floating_point():
        t.fill_(float("nan"))
    elif t.is_contiguous():
        t.view(torch.uint8).fill_(0xA5)
    else:
        t.fill_(-0x5A5A5A5B if t.element_size() >= 4 else -0x5A5B)
    return t


@pytest.fixture(autouse=True)
def _poison_gpu_allocations(request, monkeypatch):
    if "gpu" not in request.keywords:
        yield
        return
    import torch

    real_empty, real_empty_like = torch.empty, torch.empty_like

    def empty(*args, **kwargs):
        return poison_(real_empty(*args, **kwargs))

    def empty_like(*args, **kwargs):
        return poison_(real_empty_like(*args, **kwargs))

    monkeypatch.setattr(torch, "empty", empty)
    monkeypatch.setattr(torch, "empty_like", empty_like)
    yield
