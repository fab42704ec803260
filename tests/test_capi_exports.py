"""CPU-side checks of the C ABI: the built library loads without a GPU and
exports every entry point include/vm_hip.h declares."""
from __future__ import annotations

import ctypes
import os
import re

import velomind_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str) -> list[str]:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vm_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_surface():
    assert _declared("vm_hip.h") == sorted(velomind_hip.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(velomind_hip.LIB_PATH)
    missing = [s for s in _declared("vm_hip.h") if not hasattr(lib, s)]
    assert not missing, missing


def test_abi_version_without_gpu():
    assert velomind_hip.open_library().vm_hip_abi_version() == 1
