"""Test configuration: the ``gpu`` marker and shared helpers.

GPU tests run on an MI355X through the C ABI of libmolt_amd.so and compare
against the CPU oracle (``oracle/nf4_oracle.py``). They are skipped only where
torch sees no GPU at all; on a GPU box a missing library fails them loudly."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X, gfx950)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible to torch")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
