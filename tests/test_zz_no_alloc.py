"""vm_hip_qmm_f32_noalloc (the entry point that allocates nothing) against
vm_hip_qmm_f32 through the C ABI.

Both run the same kernels; the no-allocation one keeps its split-K scratch
in a static device array, so the two must agree bit for bit, and both stay
within the north-star bound of the oracle.  Each case makes two calls in a
row, the second on a smaller input, so that the second call finds the
scratch as the first left it.  A shape whose scratch would exceed the
array is refused with VM_HIP_EINVAL, and the entry point still works after.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _problem(seed: int, m: int, k: int, n: int, quant: int):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    if quant == O.QUANT_INT4:
        codes, scales = O.quantize_int4(w, 32)
        codes = codes.view(np.int8)
        block = 32
    else:
        codes, scales = O.quantize_int8(w)
        block = 0
    return a, codes, scales, block


def _both(hip, a, codes, scales, k, quant, block, stream=None):
    m, n = a.shape[0], codes.shape[1]
    da = hip.DeviceBuffer.from_array(a)
    dw = hip.DeviceBuffer.from_array(codes)
    ds = hip.DeviceBuffer.from_array(scales)
    c_ref = hip.DeviceBuffer(m * n * 4)
    c_new = hip.DeviceBuffer(m * n * 4)
    hip.qmm_f32(da.addr, dw.addr, ds.addr, c_ref.addr, m, k, n, quant, block, stream)
    hip.qmm_f32_noalloc(da.addr, dw.addr, ds.addr, c_new.addr, m, k, n, quant, block, stream)
    if stream is not None:
        stream.synchronize()
    hip.synchronize()
    return c_ref.download(np.float32, (m, n)), c_new.download(np.float32, (m, n))


def _check(hip, seed, m, k, n, quant, stream=None):
    print(f"no-alloc case seed={seed} m={m} k={k} n={n} quant={quant}", flush=True)
    a, codes, scales, block = _problem(seed, m, k, n, quant)
    ref_c, new_c = _both(hip, a, codes, scales, k, quant, block, stream)
    assert np.array_equal(ref_c, new_c), float(np.abs(ref_c - new_c).max())
    oracle = O.qmm(a, codes, scales, k, quant, block)
    err = float(np.abs(new_c - oracle).max())
    assert err <= 1e-3 * float(np.abs(oracle).max()), err


@pytest.mark.parametrize("first,second", [
    # final-output GEMV, pair-word tree across K splits (gate/up, then q/o)
    ((1, 2048, 5632, O.QUANT_INT4), (1, 2048, 2048, O.QUANT_INT4)),
    # four activation rows, eight K splits (the deepest tree of the decode shapes)
    ((4, 5632, 2048, O.QUANT_INT4), (2, 2048, 256, O.QUANT_INT4)),
    # MFMA GEMM with split-K partials and tile tickets
    ((16, 2048, 5632, O.QUANT_INT8), (8, 1024, 2048, O.QUANT_INT8)),
    ((32, 2048, 5632, O.QUANT_INT4), (16, 2048, 2048, O.QUANT_INT4)),
])
def test_noalloc_matches_qmm_f32_twice(hip, first, second):
    _check(hip, 11, *first)
    _check(hip, 12, *second)


def test_noalloc_on_a_stream_then_null_stream(hip):
    s = hip.Stream()
    try:
        _check(hip, 21, 1, 2048, 5632, O.QUANT_INT4, stream=s)
        _check(hip, 22, 16, 2048, 2048, O.QUANT_INT8, stream=s)
    finally:
        s.close()
    _check(hip, 23, 1, 576, 1536, O.QUANT_INT8)


def test_noalloc_refuses_scratch_beyond_its_array(hip, monkeypatch):
    # 130 rows INT4 at K=4096 forced to sixteen K splits of the wide kernel
    # (the tuning override) take 16 x 130 x 8192 fp32 partials (65 MiB),
    # more than the 14 MiB the static array holds.
    m, k, n = 130, 4096, 8192
    da = hip.DeviceBuffer(m * k * 4)
    dw = hip.DeviceBuffer(k // 2 * n)
    ds = hip.DeviceBuffer(k // 32 * n * 4)
    dc = hip.DeviceBuffer(m * n * 4)
    sentinel = np.full((m, n), 7.25, np.float32)
    dc.upload(sentinel)
    monkeypatch.setenv("VELOMIND_GEMM_WIDE", "128,64,16,2,1")
    with pytest.raises(hip.VmHipError) as info:
        hip.qmm_f32_noalloc(da.addr, dw.addr, ds.addr, dc.addr, m, k, n, O.QUANT_INT4, 32)
    monkeypatch.delenv("VELOMIND_GEMM_WIDE")
    assert info.value.status == hip.EINVAL
    assert "static scratch" in str(info.value)
    hip.synchronize()
    # a refused call leaves the output unwritten
    assert np.array_equal(dc.download(np.float32, (m, n)), sentinel)
    # the entry point keeps working after a refusal
    _check(hip, 31, 16, 2048, 5632, O.QUANT_INT4)
