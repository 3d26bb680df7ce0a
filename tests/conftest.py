"""Shared test setup: the `gpu` marker, the repo root on sys.path, and small helpers.

`-m "not gpu"` runs on any CPU host (the oracle pins, the host logic, the C-ABI symbol table);
`-m gpu` runs the parity tests through the HIP library on an MI355X.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def rel_err(a, b) -> float:
    """max|a - b| / max(max|b|, 1e-3): the per-tensor relative error the reference's bf16 kernel
    tests use (tests/test_flash_relation.py:84-85)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-3))


@pytest.fixture
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda")
