"""The platform hand-off diagnostic (vm_hip_diag_handoff) runs every mode
on the GPU and rejects bad arguments."""
from __future__ import annotations

import ctypes

import pytest

pytestmark = pytest.mark.gpu


def _run(lib, mode, parts, kb, rounds=50):
    us, gbs = ctypes.c_double(0.0), ctypes.c_double(0.0)
    rc = lib.vm_hip_diag_handoff(mode, parts, kb, rounds, ctypes.byref(us), ctypes.byref(gbs), None)
    return rc, us.value, gbs.value


@pytest.mark.parametrize("mode,parts,kb", [(0, 16, 0), (1, 16, 0), (2, 16, 8), (3, 16, 1)])
def test_diag_modes(hip, mode, parts, kb):
    lib = hip.open_library()
    print(f"case diag mode={mode} participants={parts} kb={kb}", flush=True)
    rc, us, gbs = _run(lib, mode, parts, kb)
    assert rc == 0, lib.vm_hip_last_error().decode()
    assert 0.0 < us < 1000.0
    if mode != 0:
        assert gbs > 0.0


def test_diag_rejects_bad_arguments(hip):
    lib = hip.open_library()
    assert _run(lib, 9, 16, 0)[0] == hip.EINVAL        # unknown mode
    assert _run(lib, 0, 1, 0)[0] == hip.EINVAL         # fewer than two participants
    assert _run(lib, 3, 16, 5)[0] == hip.EINVAL        # more than four streaming waves
    assert _run(lib, 0, 16, 0, rounds=1)[0] == hip.EINVAL
