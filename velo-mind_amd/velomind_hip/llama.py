"""ctypes binding of the LLaMA inference C ABI of libvelomind.so
(include/vm_llama.h): fp32 weights resident on the GPU, and two engines
over them -- the reference engine's per-step Graph on DeviceType::HIP
(ENGINE_GRAPH) and the resident HIP decoder (ENGINE_RESIDENT)."""
from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint64, c_void_p

import numpy as np

from . import CORE_LIB_PATH, load as _load_vmhip

ENGINE_GRAPH, ENGINE_RESIDENT = 0, 1
DECODE_GRAPH, DECODE_PER_OP, DECODE_SLICES, DECODE_PERSISTENT = 0, 1, 2, 3
W_EMBED, W_FINAL_NORM, W_LM_HEAD, W_ATTN_NORM, W_FFN_NORM = 0, 1, 2, 3, 4
W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN = 5, 6, 7, 8, 9, 10, 11

_lib = None


class LlamaConfigC(ctypes.Structure):
    _fields_ = [("vocab_size", c_int64), ("hidden_size", c_int64), ("intermediate_size", c_int64),
                ("num_layers", c_int64), ("num_heads", c_int64), ("num_kv_heads", c_int64),
                ("rms_norm_eps", c_float), ("rope_theta", c_float)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _load_vmhip()  # requires the GPU and loads libvmhip.so first
        L = ctypes.CDLL(CORE_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        p = c_void_p
        L.vm_llama_last_error.restype = c_char_p
        L.vm_llama_weights_create.argtypes = [POINTER(LlamaConfigC), POINTER(c_void_p)]
        L.vm_llama_weights_set.argtypes = [p, c_int, c_int64, p, c_int64]
        L.vm_llama_weights_fill_synthetic.argtypes = [p, c_uint64, c_float]
        L.vm_llama_weights_tie_lm_head.argtypes = [p]
        L.vm_llama_weights_destroy.argtypes = [p]
        L.vm_llama_weights_destroy.restype = None
        L.vm_llama_session_create.argtypes = [p, c_int, c_int, c_int, c_int, c_int64, POINTER(c_void_p)]
        L.vm_llama_session_destroy.argtypes = [p]
        L.vm_llama_session_destroy.restype = None
        L.vm_llama_prefill.argtypes = [p, p, c_int64, p]
        L.vm_llama_forward_step.argtypes = [p, c_int32, c_int64, p]
        L.vm_llama_generate.argtypes = [p, p, c_int64, c_int64, c_int, p, p]
        L.vm_llama_pack.argtypes = [p, c_int, c_int, POINTER(c_void_p)]
        L.vm_llama_packed_save.argtypes = [p, c_char_p]
        L.vm_llama_packed_config.argtypes = [c_char_p, POINTER(LlamaConfigC)]
        L.vm_llama_packed_load.argtypes = [c_char_p, POINTER(LlamaConfigC), POINTER(c_void_p)]
        L.vm_llama_packed_destroy.argtypes = [p]
        L.vm_llama_packed_destroy.restype = None
        L.vm_llama_session_create_packed.argtypes = [p, c_int64, POINTER(c_void_p)]
        L.vm_llama_session_decode_path.argtypes = [p, POINTER(c_int)]
        L.vm_llama_session_step_timing.argtypes = [p, p]
        for name in ("vm_llama_weights_create", "vm_llama_weights_set", "vm_llama_weights_fill_synthetic",
                     "vm_llama_weights_tie_lm_head",
                     "vm_llama_session_create", "vm_llama_prefill", "vm_llama_forward_step", "vm_llama_generate",
                     "vm_llama_pack", "vm_llama_packed_save", "vm_llama_packed_config", "vm_llama_packed_load",
                     "vm_llama_session_create_packed", "vm_llama_session_decode_path",
                     "vm_llama_session_step_timing"):
            getattr(L, name).restype = c_int
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().vm_llama_last_error().decode())


class Weights:
    """fp32 weights on the GPU in the graph's [in, out] layout."""

    def __init__(self, cfg):
        self.cfg = cfg
        c = _config_c(cfg)
        self.handle = c_void_p(None)
        _check(lib().vm_llama_weights_create(byref(c), byref(self.handle)))

    def set(self, kind: int, layer: int, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr, np.float32)
        _check(lib().vm_llama_weights_set(self.handle, kind, layer, a.ctypes.data, a.size))

    def fill_synthetic(self, seed: int, stddev: float) -> None:
        _check(lib().vm_llama_weights_fill_synthetic(self.handle, seed, stddev))

    def tie_lm_head(self) -> None:
        """lm_head := embedding^T (tied embeddings)."""
        _check(lib().vm_llama_weights_tie_lm_head(self.handle))

    @classmethod
    def from_oracle(cls, cfg, w) -> "Weights":
        """Uploads the fp32 linears of an oracle LlamaWeights."""
        out = cls(cfg)
        out.set(W_EMBED, 0, w.embed)
        out.set(W_FINAL_NORM, 0, w.final_norm)
        out.set(W_LM_HEAD, 0, w.lm_head.w)
        for layer in range(cfg.num_layers):
            out.set(W_ATTN_NORM, layer, w.attn_norm[layer])
            out.set(W_FFN_NORM, layer, w.ffn_norm[layer])
            for kind, name in ((W_Q, "wq"), (W_K, "wk"), (W_V, "wv"), (W_O, "wo"), (W_GATE, "gate"),
                               (W_UP, "up"), (W_DOWN, "down")):
                out.set(kind, layer, getattr(w, name)[layer].w)
        return out

    def close(self) -> None:
        if self.handle.value:
            lib().vm_llama_weights_destroy(self.handle)
            self.handle = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _config_c(cfg) -> LlamaConfigC:
    return LlamaConfigC(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_layers, cfg.num_heads,
                        cfg.num_kv_heads, cfg.rms_norm_eps, cfg.rope_theta)


class PackedWeights:
    """Every linear packed once on the GPU (quant.cpp layout), savable to and
    loadable from a safetensors file of I8 codes and F32 scales."""

    def __init__(self, cfg, handle: c_void_p):
        self.cfg = cfg
        self.handle = handle

    @classmethod
    def pack(cls, weights: Weights, quant_type: int, block_size: int = 0) -> "PackedWeights":
        h = c_void_p(None)
        _check(lib().vm_llama_pack(weights.handle, quant_type, block_size, byref(h)))
        return cls(weights.cfg, h)

    @staticmethod
    def file_config(path: str) -> LlamaConfigC:
        c = LlamaConfigC()
        _check(lib().vm_llama_packed_config(str(path).encode(), byref(c)))
        return c

    @classmethod
    def load(cls, path: str, cfg=None) -> "PackedWeights":
        """Loads a packed file; `cfg` defaults to the config the file records."""
        c = _config_c(cfg) if cfg is not None else cls.file_config(path)
        h = c_void_p(None)
        _check(lib().vm_llama_packed_load(str(path).encode(), byref(c), byref(h)))
        return cls(cfg if cfg is not None else c, h)

    def save(self, path: str) -> None:
        _check(lib().vm_llama_packed_save(self.handle, str(path).encode()))

    def close(self) -> None:
        if self.handle.value:
            lib().vm_llama_packed_destroy(self.handle)
            self.handle = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    def __init__(self, weights: Weights, engine: int, quant_type: int, block_size: int = 0,
                 fused_attention: bool = False, max_seq: int = 0):
        self.weights = weights
        self.vocab = weights.cfg.vocab_size
        self.handle = c_void_p(None)
        _check(lib().vm_llama_session_create(weights.handle, engine, quant_type, block_size, int(fused_attention),
                                             max_seq, byref(self.handle)))

    @classmethod
    def from_packed(cls, packed: PackedWeights, max_seq: int) -> "Session":
        """A resident-decoder session over pre-packed weights (no packing)."""
        s = cls.__new__(cls)
        s.weights = packed
        s.vocab = int(packed.cfg.vocab_size)
        s.handle = c_void_p(None)
        _check(lib().vm_llama_session_create_packed(packed.handle, max_seq, byref(s.handle)))
        return s

    def prefill(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32)
        _check(lib().vm_llama_prefill(self.handle, t.ctypes.data, t.size, out.ctypes.data))
        return out

    def forward_step(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        _check(lib().vm_llama_forward_step(self.handle, int(token), int(pos), out.ctypes.data))
        return out

    def generate(self, prompt, steps: int, use_hip_graph: bool = True):
        """Returns (steps + 1 tokens, (prefill_s, decode_s, decode_steps_timed))."""
        t = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(steps + 1, np.int32)
        timing = np.zeros(3, np.float64)
        _check(lib().vm_llama_generate(self.handle, t.ctypes.data, t.size, steps, int(use_hip_graph),
                                       out.ctypes.data, timing.ctypes.data))
        return out, (float(timing[0]), float(timing[1]), int(timing[2]))

    def step_timing(self) -> dict:
        """Graph engine: host milliseconds per decode step since the last
        prefill, split into graph construction, Graph::build, execute,
        readback, teardown (destroying a step's Executable and Graph) and the
        wait for the helper thread that builds the next step's Graph while a
        step runs (construction, build and teardown are then its time,
        overlapped with execute)."""
        t = np.zeros(7, np.float64)
        _check(lib().vm_llama_session_step_timing(self.handle, t.ctypes.data))
        n = max(1.0, t[4])
        return {"steps": int(t[4]), "construct_ms": t[0] / n * 1e3, "build_ms": t[1] / n * 1e3,
                "execute_ms": t[2] / n * 1e3, "readback_ms": t[3] / n * 1e3, "teardown_ms": t[5] / n * 1e3,
                "wait_ms": t[6] / n * 1e3}

    def decode_path(self) -> int:
        """DECODE_GRAPH / _PER_OP / _SLICES / _PERSISTENT."""
        v = c_int(-1)
        _check(lib().vm_llama_session_decode_path(self.handle, byref(v)))
        return v.value

    def close(self) -> None:
        if self.handle.value:
            lib().vm_llama_session_destroy(self.handle)
            self.handle = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
