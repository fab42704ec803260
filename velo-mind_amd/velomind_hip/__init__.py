"""ctypes binding of libvmhip.so, the C ABI declared in include/vm_hip.h.

This is a thin host-side shim used by tests, bench.py and smoke(): device
memory comes from vm_hip_malloc, every call checks the returned status and
raises ``VmHipError`` with vm_hip_last_error() text.  There is no CPU
fallback: if the library or the GPU is missing, ``load()`` raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvmhip.so")
CORE_LIB_PATH = os.path.join(_HERE, "libvelomind.so")

QUANT_INT8 = 1
QUANT_INT4 = 2
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 4, 5
EINVAL, EUNSUPPORTED, EINJECTED, ENODEVICE = -1, -2, -3, -4
A_FP32, A_ROWS, A_PIECES = 0, 1, 2   # prefill GEMM activation layouts (vm_hip_qmm_a_layout)

_lib: ctypes.CDLL | None = None


class VmHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


class GemvSrc(ctypes.Structure):
    """vm_hip_gemv_src (include/vm_hip.h)."""
    _fields_ = [("kind", c_int), ("slices", c_int), ("act", c_void_p), ("delta", c_void_p), ("norm_w", c_void_p),
                ("h_out", c_void_p), ("ss_out", c_void_p), ("ss_in", c_void_p), ("ss_count", c_int),
                ("ss_dim", c_float), ("eps", c_float), ("pos", c_void_p), ("head_dim", c_int), ("chunk", c_int),
                ("chunks", c_int), ("max_seq", c_int)]


class Prefetch(ctypes.Structure):
    """vm_hip_prefetch (include/vm_hip.h)."""
    _fields_ = [("ptr", c_void_p * 4), ("bytes", ctypes.c_uint64 * 4), ("count", c_int)]


class QmmMember(ctypes.Structure):
    """vm_hip_qmm_member (include/vm_hip.h)."""
    _fields_ = [("codes", c_void_p), ("scales", c_void_p), ("c", c_void_p), ("n", c_int64)]


def _declare(L: ctypes.CDLL) -> None:
    p = c_void_p
    sig = {
        "vm_hip_abi_version": ([], c_int),
        "vm_hip_last_error": ([], c_char_p),
        "vm_hip_device_count": ([POINTER(c_int)], c_int),
        "vm_hip_set_device": ([c_int], c_int),
        "vm_hip_get_device": ([POINTER(c_int)], c_int),
        "vm_hip_device_synchronize": ([], c_int),
        "vm_hip_malloc": ([POINTER(c_void_p), c_size_t], c_int),
        "vm_hip_free": ([p], c_int),
        "vm_hip_memcpy_h2d": ([p, p, c_size_t, p], c_int),
        "vm_hip_memcpy_d2h": ([p, p, c_size_t, p], c_int),
        "vm_hip_memcpy_d2d": ([p, p, c_size_t, p], c_int),
        "vm_hip_stream_create": ([POINTER(c_void_p)], c_int),
        "vm_hip_stream_destroy": ([p], c_int),
        "vm_hip_stream_synchronize": ([p], c_int),
        "vm_hip_event_create": ([POINTER(c_void_p)], c_int),
        "vm_hip_event_destroy": ([p], c_int),
        "vm_hip_event_record": ([p, p], c_int),
        "vm_hip_event_synchronize": ([p], c_int),
        "vm_hip_event_elapsed_ms": ([POINTER(c_float), p, p], c_int),
        "vm_hip_stream_begin_capture": ([p], c_int),
        "vm_hip_stream_end_capture": ([p, POINTER(c_void_p)], c_int),
        "vm_hip_graph_launch": ([p, p], c_int),
        "vm_hip_graph_destroy": ([p], c_int),
        "vm_hip_qmm_f32": ([p, p, p, p, c_int64, c_int64, c_int64, c_int, c_int, p], c_int),
        "vm_hip_qmm_f32_noalloc": ([p, p, p, p, c_int64, c_int64, c_int64, c_int, c_int, p], c_int),
        "vm_hip_qmm_group_f32": ([p, c_int64, c_int64, POINTER(QmmMember), c_int, c_int, c_int, p], c_int),
        "vm_hip_decode_trace_read": ([p, c_int64], c_int),
        "vm_hip_gemv_trace_read": ([p, c_int64], c_int),
        "vm_hip_qmm_add_f32": ([p, p, p, p, p, c_int64, c_int64, c_int64, c_int, c_int, p], c_int),
        "vm_hip_copy_strided": ([p, p, p, p, p, c_int, c_int, p], c_int),
        "vm_hip_attention_decode_chain_f32": ([p, p, p, p, c_int64, c_int64, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_rope_append_f32": ([p] * 10 + [c_int64] * 5 + [p], c_int),
        "vm_hip_qmm_swiglu_add_f32": ([p, p, p, p, p, p, c_int64, c_int64, c_int64, c_int, c_int, p], c_int),
        "vm_hip_qmm_norm_group_f32": ([p, p, c_float, c_int64, c_int64, POINTER(QmmMember), c_int, c_int, c_int, p],
                                      c_int),
        "vm_hip_qmm": ([p, c_int, p, p, c_int, p, c_int, c_int64, c_int64, c_int64, c_int, c_int, p], c_int),
        "vm_hip_pack_int8": ([p, p, p, c_int64, c_int64, p], c_int),
        "vm_hip_pack_int4": ([p, p, p, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_dequant_int8": ([p, p, p, c_int64, c_int64, p], c_int),
        "vm_hip_dequant_int4": ([p, p, p, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_half_to_f32": ([p, c_int, p, c_int64, p], c_int),
        "vm_hip_embedding_f32": ([p, c_int64, c_int64, p, c_int64, p, p], c_int),
        "vm_hip_rmsnorm_f32": ([p, p, p, c_int64, c_int64, c_float, p], c_int),
        "vm_hip_rope_f32": ([p, p, p, p, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_transpose_f32": ([p, p, c_int, p, p, p], c_int),
        "vm_hip_slice_f32": ([p, p, c_int, p, p, p, p, p], c_int),
        "vm_hip_concat_f32": ([p, p, p, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_repeat_kv_f32": ([p, p, c_int64, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_elementwise_f32": ([c_int, p, p, p, c_int64, p], c_int),
        "vm_hip_softmax_f32": ([p, p, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_matmul_f32": ([p, p, p, c_int64, c_int64, c_int64, c_int64, p], c_int),
        "vm_hip_attention_f32": ([p, p, p, p] + [c_int64] * 7 + [c_float, c_int, p], c_int),
        "vm_hip_fill_normal_f32": ([p, c_int64, ctypes.c_uint64, c_float, c_float, p], c_int),
        "vm_hip_add_rmsnorm_f32": ([p, p, p, p, c_int64, c_int64, c_float, p], c_int),
        "vm_hip_rope_kv_append_f32": ([p, c_int64, p, p, p, p, p, p] + [c_int64] * 4 + [p], c_int),
        "vm_hip_attention_decode_f32": ([p, p, p, p, p] + [c_int64] * 4 + [c_float, p], c_int),
        "vm_hip_attention_prefill_f32": ([p, p, p, p, p] + [c_int64] * 5 + [c_float, p], c_int),
        "vm_hip_silu_mul_f32": ([p, p, c_int64, c_int64, p], c_int),
        "vm_hip_argmax_f32": ([p, c_int64, p, p, p, c_int64, p], c_int),
        "vm_hip_memcpy_2d_d2d": ([p, c_size_t, p, c_size_t, c_size_t, c_size_t, p], c_int),
        "vm_hip_gemv_slices_count": ([c_int64, c_int64, c_int, c_int, c_int, POINTER(c_int)], c_int),
        "vm_hip_qmm_gemv_slices_f32": ([p, c_int, c_int64, p, p, p, c_int64, c_int64, c_int, c_int, c_int, p], c_int),
        "vm_hip_add_rmsnorm_slices_f32": ([p, p, c_int64, p, p, c_int64, c_float, p], c_int),
        "vm_hip_rope_kv_append_slices_f32": ([p, c_int64, p, p, p, p, p, p] + [c_int64] * 4 + [p], c_int),
        "vm_hip_argmax_slices_f32": ([p, c_int64, c_int64, p, p, p, c_int64, p], c_int),
        "vm_hip_slices_sum_f32": ([p, c_int64, c_int64, p, p], c_int),
        "vm_hip_qmm_gemv_slices_src_f32": ([POINTER(GemvSrc), p, p, p, c_int64, c_int64, c_int, c_int, c_int, p],
                                           c_int),
        "vm_hip_attention_decode_chunks": ([c_int64, c_int64, POINTER(c_int), POINTER(c_int)], c_int),
        "vm_hip_attention_decode_slices_f32": ([p, c_int64, p, c_int64, c_float, c_float, p, p, p, p, p, p,
                                                c_int64, c_int64, c_int64, c_int64, c_float, p], c_int),
        "vm_hip_slices_sum_scaled_f32": ([p, c_int64, c_int64, p, c_int64, c_float, c_float, p, p], c_int),
        "vm_hip_argmax_workspace_bytes": ([c_int64], c_int64),
        "vm_hip_argmax_slices_ws_f32": ([p, c_int64, c_int64, p, p, p, c_int64, p, c_int64, p], c_int),
        "vm_hip_attention_decode_slices_prefetch_f32": ([p, c_int64, p, c_int64, c_float, c_float, p, p, p, p, p, p,
                                                         c_int64, c_int64, c_int64, c_int64, c_float,
                                                         POINTER(Prefetch), p], c_int),
        "vm_hip_qmm_a_layout": ([c_int64, c_int64, c_int64, c_int, c_int, POINTER(c_int), POINTER(c_int64)], c_int),
        "vm_hip_qmm_staged_f32": ([p, p, p, p, c_int64, c_int64, c_int64, c_int, c_int, p], c_int),
        "vm_hip_add_rmsnorm_stage_f32": ([p, p, p, p, c_int, p, c_int64, c_int64, c_float, p], c_int),
        "vm_hip_silu_mul_stage_f32": ([p, p, c_int, p, c_int64, c_int64, p], c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def exported_symbols() -> list[str]:
    """Entry points that include/vm_hip.h declares."""
    return ["vm_hip_abi_version", "vm_hip_last_error", "vm_hip_device_count", "vm_hip_set_device",
            "vm_hip_get_device", "vm_hip_device_synchronize", "vm_hip_malloc", "vm_hip_free",
            "vm_hip_memcpy_h2d", "vm_hip_memcpy_d2h", "vm_hip_memcpy_d2d", "vm_hip_stream_create",
            "vm_hip_stream_destroy", "vm_hip_stream_synchronize", "vm_hip_event_create",
            "vm_hip_event_destroy", "vm_hip_event_record", "vm_hip_event_synchronize",
            "vm_hip_event_elapsed_ms", "vm_hip_stream_begin_capture", "vm_hip_stream_end_capture",
            "vm_hip_graph_launch", "vm_hip_graph_destroy", "vm_hip_qmm_f32", "vm_hip_qmm_f32_noalloc", "vm_hip_qmm_group_f32", "vm_hip_qmm",
            "vm_hip_pack_int8",
            "vm_hip_pack_int4", "vm_hip_dequant_int8", "vm_hip_dequant_int4", "vm_hip_half_to_f32",
            "vm_hip_embedding_f32", "vm_hip_rmsnorm_f32", "vm_hip_rope_f32", "vm_hip_transpose_f32",
            "vm_hip_slice_f32", "vm_hip_concat_f32", "vm_hip_repeat_kv_f32", "vm_hip_elementwise_f32",
            "vm_hip_softmax_f32", "vm_hip_matmul_f32", "vm_hip_attention_f32", "vm_hip_fill_normal_f32",
            "vm_hip_add_rmsnorm_f32", "vm_hip_rope_kv_append_f32", "vm_hip_attention_decode_f32",
            "vm_hip_attention_prefill_f32", "vm_hip_silu_mul_f32", "vm_hip_argmax_f32", "vm_hip_memcpy_2d_d2d",
            "vm_hip_gemv_slices_count", "vm_hip_qmm_gemv_slices_f32", "vm_hip_add_rmsnorm_slices_f32",
            "vm_hip_rope_kv_append_slices_f32", "vm_hip_argmax_slices_f32", "vm_hip_slices_sum_f32",
            "vm_hip_qmm_gemv_slices_src_f32", "vm_hip_attention_decode_chunks", "vm_hip_attention_decode_slices_f32",
            "vm_hip_slices_sum_scaled_f32", "vm_hip_attention_decode_slices_prefetch_f32",
            "vm_hip_argmax_workspace_bytes", "vm_hip_argmax_slices_ws_f32", "vm_hip_decode_workspace_bytes",
            "vm_hip_decode_step", "vm_hip_decode_status", "vm_hip_decode_trace_read", "vm_hip_gemv_trace_read",
            "vm_hip_qmm_add_f32", "vm_hip_attention_decode_chain_f32", "vm_hip_rope_append_f32",
            "vm_hip_qmm_norm_group_f32", "vm_hip_qmm_swiglu_add_f32",
            "vm_hip_qmm_a_layout", "vm_hip_qmm_staged_f32", "vm_hip_add_rmsnorm_stage_f32",
            "vm_hip_silu_mul_stage_f32", "vm_hip_copy_strided"]


def open_library() -> ctypes.CDLL:
    """dlopen libvmhip.so without touching the GPU (safe on CPU-only hosts)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libvmhip.so not built at {LIB_PATH}; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _declare(L)
        _lib = L
    return _lib


def load() -> ctypes.CDLL:
    """Open the library and require a visible gfx950 device."""
    L = open_library()
    n = c_int(0)
    check(L.vm_hip_device_count(byref(n)))
    if n.value < 1:
        raise VmHipError(ENODEVICE, "no gfx950 device visible to libvmhip")
    return L


def check(status: int) -> None:
    if status != 0:
        msg = open_library().vm_hip_last_error()
        raise VmHipError(status, msg.decode() if msg else "")


def last_error() -> str:
    msg = open_library().vm_hip_last_error()
    return msg.decode() if msg else ""


class DeviceBuffer:
    """A device allocation owned by Python (freed on close / GC)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = c_void_p(None)
        check(load().vm_hip_malloc(byref(self.ptr), self.nbytes))

    @classmethod
    def from_array(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        return buf

    @property
    def addr(self) -> int:
        return self.ptr.value or 0

    def upload(self, arr: np.ndarray, stream=None) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(open_library().vm_hip_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes, stream))

    def download(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(open_library().vm_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, stream))
        return out

    def close(self) -> None:
        if self.ptr.value:
            check(open_library().vm_hip_free(self.ptr))
            self.ptr = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        self.handle = c_void_p(None)
        check(load().vm_hip_stream_create(byref(self.handle)))

    def synchronize(self) -> None:
        check(open_library().vm_hip_stream_synchronize(self.handle))

    def close(self) -> None:
        if self.handle.value:
            check(open_library().vm_hip_stream_destroy(self.handle))
            self.handle = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.handle = c_void_p(None)
        check(load().vm_hip_event_create(byref(self.handle)))

    def record(self, stream=None) -> None:
        check(open_library().vm_hip_event_record(self.handle, stream))

    def synchronize(self) -> None:
        check(open_library().vm_hip_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float(0.0)
        check(open_library().vm_hip_event_elapsed_ms(byref(ms), self.handle, end.handle))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle.value:
                open_library().vm_hip_event_destroy(self.handle)
        except Exception:
            pass


class Graph:
    """Launches captured on a Stream between begin() and end(), replayed by launch()."""

    def __init__(self, stream: "Stream"):
        self.stream = stream
        self.exec = c_void_p(None)

    def begin(self) -> None:
        check(open_library().vm_hip_stream_begin_capture(self.stream.handle))

    def end(self) -> None:
        check(open_library().vm_hip_stream_end_capture(self.stream.handle, byref(self.exec)))

    def launch(self) -> None:
        check(open_library().vm_hip_graph_launch(self.exec, self.stream.handle))

    def close(self) -> None:
        if self.exec.value:
            check(open_library().vm_hip_graph_destroy(self.exec))
            self.exec = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _h(stream) -> c_void_p | None:
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else stream


def qmm_f32(a: int, wq: int, scale: int, c: int, m: int, k: int, n: int, quant_type: int,
            block_size: int, stream=None) -> None:
    """vm_hip_qmm_f32 on raw device addresses."""
    check(open_library().vm_hip_qmm_f32(a, wq, scale, c, m, k, n, quant_type, block_size, _h(stream)))


def qmm_group_f32(a: int, m: int, k: int, members, quant_type: int, block_size: int, stream=None) -> None:
    """vm_hip_qmm_group_f32: members = [(codes, scales, c, n), ...] device addresses."""
    arr = (QmmMember * len(members))(*[QmmMember(w, s, c, n) for w, s, c, n in members])
    check(open_library().vm_hip_qmm_group_f32(a, m, k, arr, len(members), quant_type, block_size, _h(stream)))


def qmm_f32_noalloc(a: int, wq: int, scale: int, c: int, m: int, k: int, n: int, quant_type: int,
                    block_size: int, stream=None) -> None:
    """vm_hip_qmm_f32_noalloc on raw device addresses (static split-K scratch)."""
    check(open_library().vm_hip_qmm_f32_noalloc(a, wq, scale, c, m, k, n, quant_type, block_size, _h(stream)))


def qmm(a: int, a_dtype: int, wq: int, scale: int, scale_dtype: int, c: int, c_dtype: int, m: int,
        k: int, n: int, quant_type: int, block_size: int, stream=None) -> None:
    check(open_library().vm_hip_qmm(a, a_dtype, wq, scale, scale_dtype, c, c_dtype, m, k, n,
                                    quant_type, block_size, _h(stream)))


def pack_int8(w: int, q: int, scale: int, rows: int, cols: int, stream=None) -> None:
    check(open_library().vm_hip_pack_int8(w, q, scale, rows, cols, _h(stream)))


def pack_int4(w: int, packed: int, scale: int, rows: int, cols: int, block: int, stream=None) -> None:
    check(open_library().vm_hip_pack_int4(w, packed, scale, rows, cols, block, _h(stream)))


def dequant_int8(q: int, scale: int, w: int, rows: int, cols: int, stream=None) -> None:
    check(open_library().vm_hip_dequant_int8(q, scale, w, rows, cols, _h(stream)))


def dequant_int4(packed: int, scale: int, w: int, rows: int, cols: int, block: int, stream=None) -> None:
    check(open_library().vm_hip_dequant_int4(packed, scale, w, rows, cols, block, _h(stream)))


def synchronize() -> None:
    check(open_library().vm_hip_device_synchronize())


# ---- numpy-level conveniences (host arrays in, host arrays out) ----------

def run_qmm(a: np.ndarray, wq: np.ndarray, scale: np.ndarray, k: int, quant_type: int,
            block_size: int) -> np.ndarray:
    """Upload, run vm_hip_qmm_f32 on the null stream, download C [m, n]."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    n = wq.shape[1]
    da = DeviceBuffer.from_array(a)
    dw = DeviceBuffer.from_array(np.ascontiguousarray(wq).view(np.int8))
    ds = DeviceBuffer.from_array(np.ascontiguousarray(scale, np.float32))
    dc = DeviceBuffer(max(4, m * n * 4))
    qmm_f32(da.addr, dw.addr, ds.addr, dc.addr, m, k, n, quant_type, block_size)
    return dc.download(np.float32, (m, n))


def run_pack_int8(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    dw = DeviceBuffer.from_array(w)
    dq = DeviceBuffer(max(1, rows * cols))
    ds = DeviceBuffer(max(4, cols * 4))
    pack_int8(dw.addr, dq.addr, ds.addr, rows, cols)
    return dq.download(np.int8, (rows, cols)), ds.download(np.float32, (cols,))


def run_pack_int4(w: np.ndarray, block: int = 32):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    prow = (rows + 1) // 2
    nb = (rows + block - 1) // block
    dw = DeviceBuffer.from_array(w)
    dq = DeviceBuffer(max(1, prow * cols))
    ds = DeviceBuffer(max(4, nb * cols * 4))
    pack_int4(dw.addr, dq.addr, ds.addr, rows, cols, block)
    return dq.download(np.uint8, (prow, cols)), ds.download(np.float32, (nb, cols))


# ---- LLaMA graph operators, numpy level (one call each, null stream) ----

EW_ADD, EW_MUL, EW_SIGMOID, EW_SILU_MUL = 0, 1, 2, 3
GEMV_SRC_PLAIN, GEMV_SRC_SLICES, GEMV_SRC_SWIGLU, GEMV_SRC_NORMRES, GEMV_SRC_ATTN = 0, 1, 2, 3, 4


def _dev(a: np.ndarray, dtype=np.float32) -> DeviceBuffer:
    return DeviceBuffer.from_array(np.ascontiguousarray(a, dtype))


def _out(shape) -> DeviceBuffer:
    return DeviceBuffer(max(4, int(np.prod(shape)) * 4))


def _i64(vals) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(vals, np.int64))


def run_embedding(table: np.ndarray, idx: np.ndarray) -> np.ndarray:
    idx = np.ascontiguousarray(idx, np.int32)
    shape = idx.shape + (table.shape[1],)
    dt, di, do = _dev(table), _dev(idx.reshape(-1) if idx.size else np.zeros(1, np.int32), np.int32), _out(shape)
    check(open_library().vm_hip_embedding_f32(dt.ptr, table.shape[0], table.shape[1], di.ptr, idx.size, do.ptr, None))
    return do.download(np.float32, shape)


def run_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    dx, dw, dy = _dev(x), _dev(w), _out(x.shape)
    check(open_library().vm_hip_rmsnorm_f32(dx.ptr, dw.ptr, dy.ptr, x.size // x.shape[-1], x.shape[-1], eps, None))
    return dy.download(np.float32, x.shape)


def run_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    d = x.shape[-1]
    cos_rows = cos.shape[0] if cos.ndim >= 2 else 1
    dx, dc, ds, dy = _dev(x), _dev(cos), _dev(sin), _out(x.shape)
    check(open_library().vm_hip_rope_f32(dx.ptr, dc.ptr, ds.ptr, dy.ptr, x.size // d, d, cos_rows, None))
    return dy.download(np.float32, x.shape)


def run_transpose(x: np.ndarray, perm=None) -> np.ndarray:
    perm_eff = tuple(perm) if perm else tuple(reversed(range(x.ndim)))
    out_shape = tuple(x.shape[p] for p in perm_eff)
    dx, dy = _dev(x), _out(out_shape)
    shape = _i64(x.shape)
    perm_arr = np.ascontiguousarray(np.asarray(perm_eff, np.int32))
    check(open_library().vm_hip_transpose_f32(dx.ptr, dy.ptr, x.ndim, shape.ctypes.data,
                                              perm_arr.ctypes.data if perm else None, None))
    return dy.download(np.float32, out_shape)


def run_slice(x: np.ndarray, begins, steps, out_shape) -> np.ndarray:
    dx, dy = _dev(x), _out(out_shape)
    a, b, c, d = _i64(x.shape), _i64(begins), _i64(steps), _i64(out_shape)
    check(open_library().vm_hip_slice_f32(dx.ptr, dy.ptr, x.ndim, a.ctypes.data, b.ctypes.data, c.ctypes.data,
                                          d.ctypes.data, None))
    return dy.download(np.float32, tuple(out_shape))


def run_concat(a: np.ndarray, b: np.ndarray, axis: int) -> np.ndarray:
    axis = axis % a.ndim
    outer = int(np.prod(a.shape[:axis]))
    ab = int(np.prod(a.shape[axis:]))
    bb = int(np.prod(b.shape[axis:]))
    shape = list(a.shape)
    shape[axis] += b.shape[axis]
    da, db, dy = _dev(a), _dev(b), _out(shape)
    check(open_library().vm_hip_concat_f32(da.ptr, db.ptr, dy.ptr, outer, ab, bb, None))
    return dy.download(np.float32, tuple(shape))


def run_repeat_kv(x: np.ndarray, repeats: int, axis: int) -> np.ndarray:
    axis = axis % x.ndim
    outer = int(np.prod(x.shape[:axis]))
    inner = int(np.prod(x.shape[axis + 1:]))
    shape = list(x.shape)
    shape[axis] *= repeats
    dx, dy = _dev(x), _out(shape)
    check(open_library().vm_hip_repeat_kv_f32(dx.ptr, dy.ptr, outer, x.shape[axis], repeats, inner, None))
    return dy.download(np.float32, tuple(shape))


def run_elementwise(op: int, a: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    da, dy = _dev(a), _out(a.shape)
    db = _dev(b) if b is not None else None
    check(open_library().vm_hip_elementwise_f32(op, da.ptr, db.ptr if db else None, dy.ptr, a.size, None))
    return dy.download(np.float32, a.shape)


def run_softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    axis = axis % x.ndim
    outer = int(np.prod(x.shape[:axis]))
    inner = int(np.prod(x.shape[axis + 1:]))
    dx, dy = _dev(x), _out(x.shape)
    check(open_library().vm_hip_softmax_f32(dx.ptr, dy.ptr, outer, x.shape[axis], inner, None))
    return dy.download(np.float32, x.shape)


def run_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    batch = int(np.prod(a.shape[:-2]))
    m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
    shape = a.shape[:-1] + (n,)
    da, db, dc = _dev(a), _dev(b), _out(shape)
    check(open_library().vm_hip_matmul_f32(da.ptr, db.ptr, dc.ptr, batch, m, k, n, None))
    return dc.download(np.float32, shape)


def run_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool) -> np.ndarray:
    hq, sq, d = q.shape[-3:]
    hk, sk, dv = k.shape[-3], k.shape[-2], v.shape[-1]
    batch = int(np.prod(q.shape[:-3]))
    shape = q.shape[:-1] + (dv,)
    dq, dk, dvv, do = _dev(q), _dev(k), _dev(v), _out(shape)
    check(open_library().vm_hip_attention_f32(dq.ptr, dk.ptr, dvv.ptr, do.ptr, batch, hq, hk, sq, sk, d, dv,
                                              scale, 1 if causal else 0, None))
    return do.download(np.float32, shape)
