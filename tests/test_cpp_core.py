"""Runs the C++ host-side tests (tests/cpp, tag filter ~[gpu]) in one process:
operator contract, registries, ABI values, memory planning, build-failure
recovery and the CPU-oracle graph path."""
from __future__ import annotations

import os
import subprocess

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "velomind_tests")


def test_cpp_core_suite():
    assert os.path.exists(BIN), "tests/cpp/velomind_tests not built (run __graft_entry__.build())"
    proc = subprocess.run([BIN, "~[gpu]"], capture_output=True, text=True, timeout=300)
    print(proc.stdout[-6000:])
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert "0 failed" in proc.stdout
