"""ctypes wrapper over the CPU oracle (liboracle_qmm.so).

TEST INFRASTRUCTURE ONLY: the checker used by tests/, by
``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of bench.py.
The product library never imports this module.  Each function names the
reference routine it restates; see oracle/qmm_oracle.h for how each one is
pinned.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_size_t, c_uint16, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_qmm.so")

QUANT_NONE, QUANT_INT8, QUANT_INT4 = 0, 1, 2
F32, I32, I8, BOOL, F16, BF16 = 0, 1, 2, 3, 4, 5

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        p = c_void_p
        L.vmo_quantize_int8_per_channel.argtypes = [p, p, p, c_size_t, c_size_t]
        L.vmo_dequantize_int8_per_channel.argtypes = [p, p, p, c_size_t, c_size_t]
        L.vmo_quantize_int4_block.argtypes = [p, p, p, c_size_t, c_size_t, c_size_t]
        L.vmo_dequantize_int4_block.argtypes = [p, p, p, c_size_t, c_size_t, c_size_t]
        L.vmo_quant_metrics.argtypes = [p, p, c_size_t, p]
        L.vmo_qmm_scalar_f32.argtypes = [p, p, p, p] + [c_size_t] * 9 + [c_int, c_int]
        L.vmo_qmm_decode_int8.argtypes = [p, p, p, p] + [c_size_t] * 5 + [c_int, c_int]
        L.vmo_qmm_decode_int8.restype = c_int
        L.vmo_qmm_2d_f32.argtypes = [p, p, p, p, c_size_t, c_size_t, c_size_t, c_int, c_int]
        L.vmo_qmm_scalar_mixed.argtypes = [p, c_int, p, p, c_int, p, c_int,
                                           c_size_t, c_size_t, c_size_t, c_int, c_int]
        L.vmo_f16_to_f32.argtypes = [c_uint16]
        L.vmo_f16_to_f32.restype = c_float
        L.vmo_f32_to_f16.argtypes = [c_float]
        L.vmo_f32_to_f16.restype = c_uint16
        L.vmo_bf16_to_f32.argtypes = [c_uint16]
        L.vmo_bf16_to_f32.restype = c_float
        L.vmo_f32_to_bf16.argtypes = [c_float]
        L.vmo_f32_to_bf16.restype = c_uint16
        L.vmo_cpu_has_avx2_fma.restype = c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle operands must be C-contiguous"
    return a.ctypes.data


def quantize_int8(w: np.ndarray):
    """quant.cpp:74-104 -> (codes int8 [K,N], scales f32 [N])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.zeros((rows, cols), np.int8)
    s = np.zeros(cols, np.float32)
    lib().vmo_quantize_int8_per_channel(_ptr(w), _ptr(q), _ptr(s), rows, cols)
    return q, s


def dequantize_int8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """quant.cpp:106-123."""
    rows, cols = q.shape
    out = np.zeros((rows, cols), np.float32)
    lib().vmo_dequantize_int8_per_channel(_ptr(q), _ptr(s), _ptr(out), rows, cols)
    return out


def quantize_int4(w: np.ndarray, block: int = 32):
    """quant.cpp:125-175 -> (packed uint8 [(K+1)/2,N], scales f32 [ceil(K/block),N])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    packed = np.zeros(((rows + 1) // 2, cols), np.uint8)
    s = np.zeros(((rows + block - 1) // block, cols), np.float32)
    lib().vmo_quantize_int4_block(_ptr(w), _ptr(packed), _ptr(s), rows, cols, block)
    return packed, s


def dequantize_int4(packed: np.ndarray, s: np.ndarray, rows: int, block: int = 32) -> np.ndarray:
    """quant.cpp:177-209."""
    cols = packed.shape[1]
    out = np.zeros((rows, cols), np.float32)
    lib().vmo_dequantize_int4_block(_ptr(packed), _ptr(s), _ptr(out), rows, cols, block)
    return out


def metrics(orig: np.ndarray, recon: np.ndarray):
    """quant.cpp:26-72 -> (max_diff, rmse, snr_db, cosine_sim)."""
    o = np.ascontiguousarray(orig, np.float32).ravel()
    r = np.ascontiguousarray(recon, np.float32).ravel()
    out = np.zeros(4, np.float32)
    lib().vmo_quant_metrics(_ptr(o), _ptr(r), o.size, _ptr(out))
    return tuple(float(v) for v in out)


def qmm(a: np.ndarray, wq: np.ndarray, s: np.ndarray, k: int, quant_type: int,
        block_size: int) -> np.ndarray:
    """quantized_matmul.cpp:237-267 (the CPU backend's fp32 dispatch)."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    n = wq.shape[1]
    c = np.zeros((m, n), np.float32)
    lib().vmo_qmm_2d_f32(_ptr(a), _ptr(np.ascontiguousarray(wq)), _ptr(np.ascontiguousarray(s)),
                         _ptr(c), m, k, n, quant_type, block_size)
    return c


def qmm_scalar(a: np.ndarray, wq: np.ndarray, s: np.ndarray, k: int, quant_type: int,
               block_size: int) -> np.ndarray:
    """quantized_matmul.cpp:48-141 (scalar reference, contiguous operands)."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    n = wq.shape[1]
    c = np.zeros((m, n), np.float32)
    lib().vmo_qmm_scalar_f32(_ptr(a), _ptr(np.ascontiguousarray(wq)), _ptr(np.ascontiguousarray(s)),
                             _ptr(c), m, k, n, k, 1, n, 1, n, 1, quant_type, block_size)
    return c


def qmm_decode_int8(a: np.ndarray, wq: np.ndarray, s: np.ndarray) -> np.ndarray:
    """quantized_matmul.cpp:190-235 (M=1 streaming decode, AVX2 when present)."""
    a = np.ascontiguousarray(a, np.float32).ravel()
    k, n = wq.shape
    c = np.zeros(n, np.float32)
    ok = lib().vmo_qmm_decode_int8(_ptr(a), _ptr(np.ascontiguousarray(wq)),
                                   _ptr(np.ascontiguousarray(s)), _ptr(c), k, n, 1, n, 1,
                                   QUANT_INT8, 0)
    if not ok:
        raise RuntimeError("decode stream path not applicable")
    return c


def qmm_mixed(a: np.ndarray, a_dtype: int, wq: np.ndarray, s: np.ndarray, s_dtype: int,
              c_dtype: int, k: int, quant_type: int, block_size: int) -> np.ndarray:
    """Scalar reference for F16/BF16 activations/scales/outputs (raw uint16 for halves)."""
    a = np.ascontiguousarray(a)
    m = a.shape[0]
    n = wq.shape[1]
    c = np.zeros((m, n), np.float32 if c_dtype == F32 else np.uint16)
    lib().vmo_qmm_scalar_mixed(_ptr(a), a_dtype, _ptr(np.ascontiguousarray(wq)),
                               _ptr(np.ascontiguousarray(s)), s_dtype, _ptr(c), c_dtype,
                               m, k, n, quant_type, block_size)
    return c


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.vmo_f32_to_f16(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.uint16).reshape(np.shape(x))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.vmo_f32_to_bf16(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.uint16).reshape(np.shape(x))


def has_avx2_fma() -> bool:
    return bool(lib().vmo_cpu_has_avx2_fma())


