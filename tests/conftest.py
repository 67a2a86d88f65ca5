"""Shared fixtures.  GPU tests carry the ``gpu`` marker and run on an MI355X."""

from __future__ import annotations

import gc
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X)")


@pytest.fixture()
def rng():
    return torch.Generator().manual_seed(1234)


@pytest.fixture(autouse=True)
def _free_gpu_memory(request):
    yield
    if request.node.get_closest_marker("gpu") is not None and torch.cuda.is_available():
        gc.collect()
        torch.cuda.empty_cache()


def make_moe_inputs(n, e, h, i, g, dtype=torch.float32):
    """Same draws as the reference fixture (tests/conftest.py:40-47):
    x ~ N(0,1), w ~ N(0,1)*0.02, router ~ N(0,1)*0.1, accept ~ U(0,1)."""
    x = torch.randn(n, h, generator=g, dtype=dtype)
    w1 = torch.randn(e, i, h, generator=g, dtype=dtype) * 0.02
    w2 = torch.randn(e, h, i, generator=g, dtype=dtype) * 0.02
    w3 = torch.randn(e, i, h, generator=g, dtype=dtype) * 0.02
    router = torch.randn(e, h, generator=g, dtype=dtype) * 0.1
    accept = torch.rand(n, generator=g)
    return x, w1, w2, w3, router, accept


def bf16_bits(t: torch.Tensor):
    """uint16 numpy view of a bf16 tensor's bits (host)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view("uint16")
