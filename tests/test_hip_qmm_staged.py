"""Prefill GEMM activations staged by their producer
(vm_hip_add_rmsnorm_stage_f32, vm_hip_silu_mul_stage_f32,
vm_hip_qmm_staged_f32): the GEMM on the staged buffer equals
vm_hip_qmm_f32 on the fp32 rows the producer also writes, bit for bit, in
both layouts (row-major for the small-tile kernel, operand order for the
wide kernel) and for INT8 per column, INT8 blockwise and INT4; the fp32
rows equal the plain producers' (SiLU exactly, RMSNorm to the rounding of
its sum of squares); the oracle bounds the result as for every GEMM."""
from __future__ import annotations

from ctypes import byref, c_int, c_int64

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

A_FP32, A_ROWS, A_PIECES = 0, 1, 2


def _weights(kind, k, n, rng):
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    if kind == "int8":
        q, s = O.quantize_int8(w)
        return q, s, 1, 0, O.QUANT_INT8
    if kind == "int8_block":
        q = rng.integers(-127, 128, (k, n), dtype=np.int8)
        s = (rng.random(((k + 31) // 32, n)) * 0.01 + 1e-4).astype(np.float32)
        return q, s, 1, 32, O.QUANT_INT8
    q, s = O.quantize_int4(w, 32)
    return q, s, 2, 32, O.QUANT_INT4


def _layout(lib, rows, k, n, qt, blk):
    lay, nbytes = c_int(-1), c_int64(-1)
    assert lib.vm_hip_qmm_a_layout(rows, k, n, qt, blk, byref(lay), byref(nbytes)) == 0
    return lay.value, nbytes.value


def _gemm_both(H, lib, staged, a32, q, s, rows, k, n, qt, blk, layout):
    dq, ds = H.DeviceBuffer.from_array(q), H.DeviceBuffer.from_array(s)
    c1, c2 = H.DeviceBuffer(rows * n * 4), H.DeviceBuffer(rows * n * 4)
    H.check(lib.vm_hip_qmm_staged_f32(staged.ptr, dq.ptr, ds.ptr, c1.ptr, rows, k, n, qt, blk, None))
    H.qmm_f32(a32.addr, dq.addr, ds.addr, c2.addr, rows, k, n, qt, blk)
    return c1.download(np.float32, (rows, n)), c2.download(np.float32, (rows, n))


@pytest.mark.parametrize("rows,n,want", [(24, 1024, A_ROWS), (130, 2048, A_PIECES), (512, 2048, A_PIECES)])
@pytest.mark.parametrize("kind", ["int8", "int8_block", "int4"])
def test_add_rmsnorm_stage(hip, rows, n, want, kind):
    if kind != "int8":
        want = A_PIECES   # blockwise scales always take the wide kernel's operand order
    H, lib = hip, hip.open_library()
    k = 2048
    rng = np.random.default_rng(rows + n + len(kind))
    h = rng.standard_normal((rows, k)).astype(np.float32)
    delta = rng.standard_normal((rows, k)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    q, s, qt, blk, oq = _weights(kind, k, n, rng)
    layout, nbytes = _layout(lib, rows, k, n, qt, blk)
    assert layout == want
    print(f"case add_rmsnorm_stage rows={rows} k={k} n={n} kind={kind} layout={layout}", flush=True)
    dh, dh2 = H.DeviceBuffer.from_array(h), H.DeviceBuffer.from_array(h)
    dd, dw = H.DeviceBuffer.from_array(delta), H.DeviceBuffer.from_array(w)
    staged, hn, hn2 = H.DeviceBuffer(nbytes), H.DeviceBuffer(rows * k * 4), H.DeviceBuffer(rows * k * 4)
    H.check(lib.vm_hip_add_rmsnorm_stage_f32(dh.ptr, dd.ptr, dw.ptr, staged.ptr, layout, hn.ptr, rows, k, 1e-5, None))
    H.check(lib.vm_hip_add_rmsnorm_f32(dh2.ptr, dd.ptr, dw.ptr, hn2.ptr, rows, k, 1e-5, None))
    assert np.array_equal(dh.download(np.float32, (rows, k)), dh2.download(np.float32, (rows, k)))
    x = hn.download(np.float32, (rows, k))
    np.testing.assert_allclose(x, hn2.download(np.float32, (rows, k)), rtol=2e-6, atol=1e-6)
    out, ref_gpu = _gemm_both(H, lib, staged, hn, q, s, rows, k, n, qt, blk, layout)
    assert np.array_equal(out.view(np.uint32), ref_gpu.view(np.uint32))
    ref = O.qmm(x, q, s, k, oq, blk)
    assert np.abs(out - ref).max() <= 1e-3 * np.abs(ref).max()


@pytest.mark.parametrize("rows,inter,n,want", [(24, 2560, 960, A_ROWS), (130, 1024, 2048, A_PIECES),
                                               (512, 5632, 2048, A_PIECES)])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_silu_mul_stage(hip, rows, inter, n, want, kind):
    if kind != "int8":
        want = A_PIECES   # blockwise scales always take the wide kernel's operand order
    H, lib = hip, hip.open_library()
    rng = np.random.default_rng(rows + inter + len(kind))
    gu = rng.standard_normal((rows, 2 * inter)).astype(np.float32) * 3
    q, s, qt, blk, oq = _weights(kind, inter, n, rng)
    layout, nbytes = _layout(lib, rows, inter, n, qt, blk)
    assert layout == want
    print(f"case silu_mul_stage rows={rows} inter={inter} n={n} kind={kind} layout={layout}", flush=True)
    dg = H.DeviceBuffer.from_array(gu)
    staged, y, y2 = H.DeviceBuffer(nbytes), H.DeviceBuffer(rows * inter * 4), H.DeviceBuffer(rows * inter * 4)
    H.check(lib.vm_hip_silu_mul_stage_f32(dg.ptr, staged.ptr, layout, y.ptr, rows, inter, None))
    H.check(lib.vm_hip_silu_mul_f32(dg.ptr, y2.ptr, rows, inter, None))
    x = y.download(np.float32, (rows, inter))
    assert np.array_equal(x.view(np.uint32), y2.download(np.float32, (rows, inter)).view(np.uint32))
    out, ref_gpu = _gemm_both(H, lib, staged, y, q, s, rows, inter, n, qt, blk, layout)
    assert np.array_equal(out.view(np.uint32), ref_gpu.view(np.uint32))
    ref = O.qmm(x, q, s, inter, oq, blk)
    assert np.abs(out - ref).max() <= 1e-3 * np.abs(ref).max()


def test_stage_rows_with_extreme_magnitudes(hip):
    # rows of 1e-6, 1e5 and one holding an infinity: the staged GEMM still
    # equals vm_hip_qmm_f32 on the same rows (the exponents and the split are
    # the pre-pass's)
    H, lib = hip, hip.open_library()
    rows, inter, n = 130, 1024, 2048
    rng = np.random.default_rng(9)
    gu = rng.standard_normal((rows, 2 * inter)).astype(np.float32)
    gu[3] *= 1e-6
    gu[4, inter:] *= 1e5
    gu[5, inter + 7] = np.inf
    q, s, qt, blk, _ = _weights("int4", inter, n, rng)
    layout, nbytes = _layout(lib, rows, inter, n, qt, blk)
    dg = H.DeviceBuffer.from_array(gu)
    staged, y = H.DeviceBuffer(nbytes), H.DeviceBuffer(rows * inter * 4)
    H.check(lib.vm_hip_silu_mul_stage_f32(dg.ptr, staged.ptr, layout, y.ptr, rows, inter, None))
    out, ref_gpu = _gemm_both(H, lib, staged, y, q, s, rows, inter, n, qt, blk, layout)
    assert np.array_equal(np.isnan(out), np.isnan(ref_gpu))
    fin = ~np.isnan(out)
    assert np.array_equal(out[fin].view(np.uint32), ref_gpu[fin].view(np.uint32))


def test_stage_arguments(hip):
    H, lib = hip, hip.open_library()
    assert _layout(lib, 4, 2048, 2048, 2, 32)[0] == A_FP32     # GEMV rows take fp32 A
    assert _layout(lib, 64, 2040, 2048, 2, 32)[0] == A_FP32    # K % 32 != 0: the generic kernel
    buf = H.DeviceBuffer(1 << 20)
    x = H.DeviceBuffer(64 * 2048 * 4)
    assert lib.vm_hip_silu_mul_stage_f32(x.ptr, buf.ptr, 7, None, 8, 1024, None) == H.EINVAL
    assert lib.vm_hip_silu_mul_stage_f32(x.ptr, buf.ptr, A_ROWS, None, 8, 1000, None) == H.EINVAL
    q = H.DeviceBuffer(2048 * 2048)
    s = H.DeviceBuffer(64 * 2048 * 4)
    c = H.DeviceBuffer(512 * 2048 * 4)
    # rows the GEMM does not take, and a null staged buffer
    assert lib.vm_hip_qmm_staged_f32(buf.ptr, q.ptr, s.ptr, c.ptr, 3, 2048, 2048, 2, 32, None) == H.EINVAL
    assert lib.vm_hip_qmm_staged_f32(None, q.ptr, s.ptr, c.ptr, 512, 2048, 2048, 2, 32, None) == H.EINVAL
