"""Shared pytest configuration.

Tests marked ``@pytest.mark.gpu`` run the HIP kernels and are skipped unless a HIP
device is visible (the reference's rule, tests/conftest.py:30-36). Everything else runs
on the CPU: the oracle against its pins and golden fixtures, the argument checks of the
Python entry points, and the C-ABI library's exports (loaded, never called).
"""

from __future__ import annotations

import pytest
import torch


def gpu_available() -> bool:
    return bool(torch.cuda.is_available())


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); skipped without one")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if gpu_available():
        return
    skip_gpu = pytest.mark.skip(reason="no HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip_gpu)
