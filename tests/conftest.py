"""Shared test setup.

Markers: `gpu` — needs an MI355X (the driver runs `-m gpu` there and
`-m "not gpu"` on CPU); `slow` — long CPU checks.

The package directory mini-llm-stack_amd/ is put on sys.path so the tests
import the reference's module paths (kernels.*, serve.quantize, train.fp8),
and the repo root so they can import the CPU oracle (oracle/).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "mini-llm-stack_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")
    config.addinivalue_line("markers", "slow: long-running CPU check")


def golden(name: str):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda:0")
