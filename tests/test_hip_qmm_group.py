"""vm_hip_qmm_group_f32 (sibling quantized matmuls sharing A, one launch
for rows_m <= 4) against the oracle and against separate vm_hip_qmm_f32
calls, through the C ABI.

Bounds: every member within 1e-5 * max|C_ref| of the oracle for rows <= 4
(the fp32 GEMV bound of tests/test_hip_qmm.py; 1e-3 for the GEMM rows) and
within 1e-6 * max|C| of the separate call (the K split follows the combined width, so only the grouping of the
fp32 partial sums differs); a group of one is the separate call bit for
bit.  Shapes: TinyLlama's q | k | v and gate | up, SmolLM2's q | k | v,
rows 1..4 (one grouped launch) and 8 (one launch per member), a member
width that is not a multiple of 16 (its own kernel), and the argument
checks.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _normal(shape, seed, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def _rel(out, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(out, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def _pack(qt, k, n, seed):
    w = _normal((k, n), seed, 0.02)
    if qt == O.QUANT_INT4:
        p, s = O.quantize_int4(w, 32)
        return p.view(np.int8), s, 32
    q, s = O.quantize_int8(w)
    return q, s, 0


def _run(hip, qt, m, k, widths, seed=0):
    """Returns (grouped outputs, separate outputs, oracle outputs)."""
    mats = [_pack(qt, k, n, seed + 17 * i + n) for i, n in enumerate(widths)]
    block = mats[0][2]
    x = _normal((m, k), seed + 1)
    bufs = []

    def dev(arr):
        b = hip.DeviceBuffer.from_array(np.ascontiguousarray(arr))
        bufs.append(b)
        return b

    da = dev(x)
    members, outs_g, outs_s = [], [], []
    for (q, s, _), n in zip(mats, widths):
        dq, ds = dev(q), dev(s)
        cg = hip.DeviceBuffer(m * n * 4)
        cs = hip.DeviceBuffer(m * n * 4)
        bufs += [cg, cs]
        members.append((dq.addr, ds.addr, cg.addr, n))
        outs_g.append(cg)
        outs_s.append((dq, ds, cs, n))
    hip.qmm_group_f32(da.addr, m, k, members, qt, block)
    for dq, ds, cs, n in outs_s:
        hip.qmm_f32(da.addr, dq.addr, ds.addr, cs.addr, m, k, n, qt, block)
    hip.synchronize()
    grouped = [b.download(np.float32, (m, n)) for b, n in zip(outs_g, widths)]
    separate = [cs.download(np.float32, (m, n)) for _, _, cs, n in outs_s]
    ref = [O.qmm(x, q, s, k, qt, block) for q, s, _ in mats]
    for b in bufs:
        b.close()
    return grouped, separate, ref


SHAPES = {
    "tinyllama_qkv": (2048, (2048, 256, 256)),
    "tinyllama_gate_up": (2048, (5632, 5632)),
    "smollm2_qkv": (960, (960, 320, 320)),
    "small_four": (512, (128, 64, 256, 64)),
}


@pytest.mark.parametrize("qt", [O.QUANT_INT4, O.QUANT_INT8])
@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
def test_group_matches_oracle_and_separate_calls(hip, qt, shape, m):
    k, widths = SHAPES[shape]
    print(f"case group qt={qt} {shape} m={m}", flush=True)
    grouped, separate, ref = _run(hip, qt, m, k, widths, seed=m)
    # rows > 4 run the MFMA GEMM per member: blockwise weights staged in
    # fp16, the 1e-3 bound of tests/test_hip_qmm.py
    tol = 1e-5 if m <= 4 else 1e-3
    for g, (out, sep, r) in enumerate(zip(grouped, separate, ref)):
        assert _rel(out, r) <= tol, f"member {g}: {_rel(out, r):.2e} from the oracle"
        if m > 4:
            assert np.array_equal(out, sep), f"member {g}: per-member launches differ from vm_hip_qmm_f32"
        else:
            assert _rel(out, sep) <= 1e-6, f"member {g}: {_rel(out, sep):.2e} from the separate call"


@pytest.mark.parametrize("qt", [O.QUANT_INT4, O.QUANT_INT8])
def test_group_of_one_is_the_separate_call(hip, qt):
    grouped, separate, ref = _run(hip, qt, 1, 2048, (5632,), seed=3)
    assert np.array_equal(grouped[0], separate[0])
    assert _rel(grouped[0], ref[0]) <= 1e-5


def test_member_outside_the_gemv_runs_on_its_own(hip):
    # a width that is not a multiple of 16 needs the generic kernel: the
    # group falls back to one launch per member, results unchanged
    grouped, separate, ref = _run(hip, O.QUANT_INT8, 1, 256, (128, 100), seed=5)
    for out, sep, r in zip(grouped, separate, ref):
        assert np.array_equal(out, sep)
        assert _rel(out, r) <= 1e-5


def test_group_argument_checks(hip):
    lib = hip.open_library()
    members = (hip.QmmMember * 5)()
    assert lib.vm_hip_qmm_group_f32(None, 1, 8, members, 0, O.QUANT_INT8, 0, None) == hip.EINVAL
    assert lib.vm_hip_qmm_group_f32(None, 1, 8, members, 5, O.QUANT_INT8, 0, None) == hip.EINVAL
    # a member with a null output is refused before anything runs
    buf = hip.DeviceBuffer(1024)
    one = (hip.QmmMember * 1)(hip.QmmMember(buf.addr, buf.addr, None, 16))
    rc = lib.vm_hip_qmm_group_f32(ctypes.c_void_p(buf.addr), 1, 8, one, 1, O.QUANT_INT8, 0, None)
    assert rc == hip.EINVAL
    assert b"null output" in lib.vm_hip_last_error()
    buf.close()
