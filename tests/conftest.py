"""Shared pytest setup: import paths, the `gpu` marker, seeds and devices.

Tests marked `gpu` exercise libfa_gfx950.so on an MI355X and compare it with
the CPU oracle under /oracle; the rest run on any CPU.
"""
import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "flash-attn-mps_amd", ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libfa_gfx950.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(123)


@pytest.fixture
def device():
    return torch.device("cuda", 0)
