"""CPU-side checks of the C ABI: the built library loads without a GPU and
exports every entry point include/vm_hip.h and include/vm_llama.h declare."""
from __future__ import annotations

import ctypes
import os
import re

import velomind_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str) -> list[str]:
    with open(os.path.join(ROOT, "include", header)) as f:
        text = f.read()
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


def _declared_llama() -> list[str]:
    with open(os.path.join(ROOT, "include", "vm_llama.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vm_llama_[a-z0-9_]+)\s*\(", text)))


def test_core_library_exports_every_llama_symbol():
    ctypes.CDLL(velomind_hip.LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    lib = ctypes.CDLL(velomind_hip.CORE_LIB_PATH)
    declared = _declared_llama()
    assert "vm_llama_session_create_packed" in declared and "vm_llama_packed_load" in declared
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
