"""Shared pytest setup.

Markers:
  gpu — needs a ROCm GPU (MI355X); auto-skipped when none is visible,
        mirroring the reference's ``requires_cuda`` auto-skip
        (tests/conftest.py:55-85 of luisfuturist/catopt).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

_GPU: bool | None = None


def gpu_available() -> bool:
    global _GPU
    if _GPU is None:
        try:
            import torch

            _GPU = bool(torch.cuda.is_available()) and torch.cuda.device_count() > 0
        except Exception:  # pragma: no cover - torch import failure
            _GPU = False
    return _GPU


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (auto-skipped without one)")
    config.addinivalue_line("markers", "slow: long-running")


def pytest_collection_modifyitems(config, items):
    if any("gpu" in it.keywords for it in items) and not gpu_available():
        skip = pytest.mark.skip(reason="no ROCm GPU visible")
        for it in items:
            if "gpu" in it.keywords:
                it.add_marker(skip)


@pytest.fixture
def dev():
    import torch

    return torch.device("cuda", 0)


def pytest_runtest_setup(item):
    # Name the case before any GPU work so a fault that kills the process
    # still leaves the test id in the log.
    if "gpu" in item.keywords:
        print(f"\n[gpu-case] {item.nodeid}", flush=True)
        os.environ.setdefault("HSA_ENABLE_IPC_MODE_LEGACY", "0")
