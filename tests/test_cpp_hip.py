"""Runs the C++ DeviceType::HIP tests (tests/cpp, tag filter [gpu]) in one
process: graphs built with g.build(DeviceType::HIP) against the oracle,
INT4 quantize-and-bind, dtype keys, batched activations, the single-arena
memory plan, bind_input, injected failures and concurrent per-thread
streams."""
from __future__ import annotations

import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "velomind_tests")

pytestmark = pytest.mark.gpu


def test_cpp_hip_suite():
    assert os.path.exists("/dev/kfd"), "GPU test selected but /dev/kfd is absent"
    assert os.path.exists(BIN), "tests/cpp/velomind_tests not built (run __graft_entry__.build())"
    proc = subprocess.run([BIN, "[gpu]"], capture_output=True, text=True, timeout=600)
    print(proc.stdout[-8000:])
    assert proc.returncode == 0, proc.stdout[-6000:] + proc.stderr[-2000:]
    assert "0 failed" in proc.stdout and "0 skipped" in proc.stdout
