"""Shared pytest setup: markers, import paths and common fixtures."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "velo-mind_amd", os.path.join("tests", "golden")):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _gpu_present() -> bool:
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def hip():
    """The product's ctypes binding; fails loudly if the HIP library is absent."""
    import velomind_hip

    if not _gpu_present():
        pytest.fail("GPU test selected but /dev/kfd is absent")
    velomind_hip.load()
    return velomind_hip
