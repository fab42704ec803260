"""Host-side launch plans of the C ABI, checked without a GPU: which
activation layout the prefill GEMM asks its producers for
(vm_hip_qmm_a_layout), at the edges where a kernel's addressing or a
producer's row limit rules a layout out."""
from __future__ import annotations

from ctypes import byref, c_int, c_int64

import velomind_hip as H


def _layout(rows, k, n, qt=H.QUANT_INT4, blk=32):
    lib = H.open_library()
    lay, nbytes = c_int(-1), c_int64(-1)
    rc = lib.vm_hip_qmm_a_layout(rows, k, n, qt, blk, byref(lay), byref(nbytes))
    assert rc == 0, lib.vm_hip_last_error().decode()
    return lay.value, nbytes.value


def test_wide_kernel_taken_at_prefill_shapes():
    # TinyLlama's gate|up at a 512-token prompt: the wide kernel's operand order.
    assert _layout(512, 2048, 5632)[0] == H.A_PIECES
    assert _layout(512, 2048, 5632, H.QUANT_INT8, 0)[0] == H.A_PIECES


def test_blockwise_weights_always_take_the_wide_kernel():
    # Only the wide kernel applies block scales to each chunk's fp32 sum;
    # it addresses C from a 64-bit base per 128-row tile, so outputs of
    # 2 GiB and more stay on it too (tests/test_hip_qmm.py writes one).
    for rows in (5, 16, 64, 512, 4096):
        assert _layout(rows, 2048, 5632)[0] == H.A_PIECES
    assert _layout(4096, 2048, 131072)[0] == H.A_PIECES
    assert _layout(16, 2048, 5632, H.QUANT_INT8, 32)[0] == H.A_PIECES
    # per-column INT8 keeps the small-tile kernel for few rows
    assert _layout(16, 2048, 5632, H.QUANT_INT8, 0)[0] == H.A_ROWS


def test_rows_longer_than_the_producers_limit_take_fp32():
    # add_rmsnorm_stage / silu_mul_stage hold a whole row (at most 6144).
    assert _layout(512, 6144, 2048)[0] != H.A_FP32
    assert _layout(512, 6400, 2048) == (H.A_FP32, 0)
    assert _layout(512, 11008, 4096, H.QUANT_INT8, 0) == (H.A_FP32, 0)
