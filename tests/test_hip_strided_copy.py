"""vm_hip_copy_strided on the GPU against numpy's strided views, bit for
bit: the gather (strided view -> contiguous) and scatter (contiguous ->
strided view) that let the HIP QuantizedMatMul take the strided A, B and C
the reference's CPU kernel honours (src/cpu/ops/quantized_matmul.cpp:306-315).
Element widths 1, 2 and 4, ranks 1 to 8, transposed, broadcast (stride 0)
reads, an empty tensor and the argument errors."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

I64 = ctypes.c_int64


def _arr(vals):
    return (I64 * max(len(vals), 1))(*vals)


def _copy(hip, dst, dst_strides, src, src_strides, shape, width):
    return hip.load().vm_hip_copy_strided(dst, _arr(dst_strides), src, _arr(src_strides), _arr(shape),
                                          len(shape), width, None)


def _elem_strides(a: np.ndarray):
    return [s // a.itemsize for s in a.strides]


CASES = [
    # (dtype, base shape, view builder)
    (np.float32, (40, 72), lambda b: b[3:35:2, 5:69:3]),
    (np.float32, (64, 48), lambda b: b.T),
    (np.int8, (33, 130), lambda b: b[:, 1:129]),
    (np.uint16, (6, 10, 12), lambda b: b.transpose(2, 0, 1)[::2]),
    (np.float32, (7,), lambda b: np.lib.stride_tricks.as_strided(b, (5, 7), (0, 4))),  # repeated rows
    (np.int8, (2,) * 8, lambda b: b.transpose(7, 6, 5, 4, 3, 2, 1, 0)),
    (np.float32, (1000,), lambda b: b[::7]),
    (np.float32, (4, 0, 3), lambda b: b.transpose(1, 0, 2)),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_gather_and_scatter_match_numpy(hip, case):
    dtype, base_shape, make = CASES[case]
    rng = np.random.default_rng(case)
    base = rng.integers(0, 255, size=base_shape).astype(dtype)
    view = make(base)
    width = view.itemsize
    shape = list(view.shape)
    offset = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // width
    print(f"case {case}: dtype {np.dtype(dtype).name} shape {shape} strides {_elem_strides(view)}", flush=True)
    d_base = hip.DeviceBuffer.from_array(base) if base.size else hip.DeviceBuffer(16)
    dense = np.ascontiguousarray(view)
    d_dense = hip.DeviceBuffer(max(dense.nbytes, 16))
    src = (d_base.addr + offset * width) if base.size else d_base.addr
    dense_strides = _elem_strides(dense) if dense.size else [0] * len(shape)
    assert _copy(hip, d_dense.addr, dense_strides, src, _elem_strides(view), shape, width) == 0, hip.last_error()
    if dense.size:
        got = d_dense.download(dtype, dense.shape)
        assert np.array_equal(got.view(np.uint8), dense.view(np.uint8))

    # scatter back into a pitched destination whose gaps hold a sentinel
    if dense.size and all(s > 0 for s in _elem_strides(view)):
        fill = np.full(base_shape, 77, dtype)
        d_out = hip.DeviceBuffer.from_array(fill)
        assert _copy(hip, d_out.addr + offset * width, _elem_strides(view), d_dense.addr, dense_strides,
                     shape, width) == 0, hip.last_error()
        want = fill.copy()
        make(want)[...] = dense
        got = d_out.download(dtype, base_shape)
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_argument_errors(hip):
    d = hip.DeviceBuffer(64)
    one = [4]
    assert _copy(hip, d.addr, one, d.addr, one, [4], 3) != 0                        # 3-byte elements
    assert _copy(hip, d.addr, [1] * 9, d.addr, [1] * 9, [1] * 9, 4) != 0          # rank 9
    assert _copy(hip, d.addr, [1], d.addr, [-1], [4], 4) != 0                       # negative stride
    assert _copy(hip, d.addr, [1], d.addr, [1], [-2], 4) != 0                       # negative dimension
    assert _copy(hip, None, [1], d.addr, [1], [4], 4) != 0                          # null destination
    assert _copy(hip, None, [1], None, [1], [0], 4) == 0                            # nothing to copy
