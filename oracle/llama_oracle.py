"""CPU oracle of the LLaMA graph around QuantizedMatMul (numpy, fp32).

TEST INFRASTRUCTURE ONLY: the checker used by tests/, ``__graft_entry__.
smoke()`` and the ``cpu_baseline`` leg of bench.py.  The product library
never imports it.

Each function restates one reference operator or graph routine and cites
it.  How each is pinned (tests/test_oracle_llama.py):

  embedding, transpose, slice_, concat      numpy's own take / transpose /
                                            basic slicing / concatenate
  repeat_kv                                 numpy.repeat along the head axis
  softmax                                   sums to 1, shift invariance,
                                            closed form on two columns
  rmsnorm                                   unit RMS output with w = 1,
                                            scale equivariance
  rope_cache, rope                          position 0 is the identity,
                                            pair norms preserved, rotation
                                            by a then b equals rotation by
                                            a + b, hand-computed 2-D case
  attention                                 one key -> that key's value;
                                            equal scores -> mean of values;
                                            GQA == repeat_kv + MHA; causal
                                            row i == non-causal attention
                                            over keys 0..sk-sq+i
  prefill / decode / load_toy_llama         HuggingFace transformers'
                                            LlamaForCausalLM on the
                                            reference's toy_llama fixture
                                            and on a random GQA config;
                                            decode after prefill == prefill
                                            over the longer prompt
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass, field

import numpy as np

import oracle as Q  # quantized matmul and packers (liboracle_qmm.so)

f32 = np.float32


# ---------------------------------------------------------------- operators

def embedding(table: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """src/cpu/ops/embedding.cpp:16-33: out[..., :] = table[idx[...], :]."""
    idx = np.asarray(idx, np.int64)
    if idx.size and (idx.min() < 0 or idx.max() >= table.shape[0]):
        raise IndexError("Embedding: index out of range (src/executable.cpp:54-66)")
    return table[idx].astype(f32)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """src/cpu/ops/rmsnorm.cpp:17-60 (last axis): x / sqrt(mean(x^2)+eps) * w,
    all in fp32."""
    x = x.astype(f32)
    ms = (x * x).sum(axis=-1, keepdims=True, dtype=f32) / f32(x.shape[-1])
    inv = f32(1.0) / np.sqrt(ms + f32(eps))
    return (x * inv * w.astype(f32)).astype(f32)


def rope_cache(seq_len: int, head_dim: int, theta: float, pos_offset: int = 0):
    """examples/common/llama/llama_rope_mask.cpp:7-24: cos/sin [seq, head_dim/2]
    with inv_freq_i = 1 / theta^(2i/head_dim) in fp32."""
    half = head_dim // 2
    i = np.arange(half, dtype=f32)
    exp_val = (f32(2) * i) / f32(head_dim)
    inv_freq = f32(1.0) / np.power(f32(theta), exp_val, dtype=f32)
    t = (np.arange(seq_len, dtype=np.int64) + pos_offset).astype(f32)
    freq = (t[:, None] * inv_freq[None, :]).astype(f32)
    return np.cos(freq).astype(f32), np.sin(freq).astype(f32)


def causal_mask(num_heads: int, seq_len: int) -> np.ndarray:
    """llama_rope_mask.cpp:27-40: -1e9 above the diagonal, 0 elsewhere."""
    m = np.where(np.arange(seq_len)[None, :] > np.arange(seq_len)[:, None], f32(-1e9), f32(0.0)).astype(f32)
    return np.broadcast_to(m, (num_heads, seq_len, seq_len)).copy()


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """src/cpu/ops/rotary_embedding.cpp:16-45: rows of head_dim; position of
    flat row i is i % cos_rows (0 when the cache has one row)."""
    d = x.shape[-1]
    h = d // 2
    rows = x.reshape(-1, d).astype(f32)
    cos2 = cos.reshape(-1, h).astype(f32)
    sin2 = sin.reshape(-1, h).astype(f32)
    n_pos = cos2.shape[0] if cos.ndim >= 2 else 1
    pos = np.arange(rows.shape[0]) % n_pos if n_pos > 1 else np.zeros(rows.shape[0], np.int64)
    c, s = cos2[pos], sin2[pos]
    a, b = rows[:, :h], rows[:, h:]
    y = np.empty_like(rows)
    y[:, :h] = a * c - b * s
    y[:, h:] = b * c + a * s
    return y.reshape(x.shape)


def transpose(x: np.ndarray, perm=None) -> np.ndarray:
    """src/cpu/ops/transpose.cpp:17-68; empty perm reverses the axes
    (shape_helpers.h:125-146)."""
    return np.ascontiguousarray(np.transpose(x, None if not perm else perm))


def slice_(x: np.ndarray, begins, ends, strides=()) -> np.ndarray:
    """src/cpu/ops/slice.cpp:21-110 with the clamping of shape_helpers.h:
    178-211: negative begin/end count from the end, both clamp to [0, dim],
    non-positive or missing strides mean 1, missing axes are kept whole."""
    sl = []
    for ax, dim in enumerate(x.shape):
        if ax < len(begins):
            b = begins[ax] + dim if begins[ax] < 0 else begins[ax]
            e = ends[ax] + dim if ends[ax] < 0 else ends[ax]
            b, e = min(max(b, 0), dim), min(max(e, 0), dim)
            st = strides[ax] if ax < len(strides) and strides[ax] > 0 else 1
            sl.append(slice(b, max(b, e), st))
        else:
            sl.append(slice(None))
    return np.ascontiguousarray(x[tuple(sl)])


def concat(a: np.ndarray, b: np.ndarray, axis: int) -> np.ndarray:
    """src/cpu/ops/concat.cpp:19-72."""
    return np.concatenate([a, b], axis=axis)


def repeat_kv(x: np.ndarray, repeats: int, axis: int = 0) -> np.ndarray:
    """src/cpu/ops/repeat_kv.cpp:20-62: output head h copies input head
    h // repeats along `axis`."""
    return np.repeat(x, repeats, axis=axis)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """src/cpu/ops/softmax.cpp:18-48: exp(x - max) / sum in fp32."""
    x = x.astype(f32)
    e = np.exp(x - x.max(axis=axis, keepdims=True))
    return (e / e.sum(axis=axis, keepdims=True, dtype=f32)).astype(f32)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """src/cpu/ops/matmul.cpp fp32 path; equal batch dims
    (shape_helpers.h:36-84)."""
    return np.matmul(a.astype(f32), b.astype(f32)).astype(f32)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float = 0.0, causal: bool = True) -> np.ndarray:
    """src/cpu/ops/fused_attention.cpp:22-138 for [..., H, S, D] operands:
    scale <= 0 means 1/sqrt(D); query head h uses KV head h // (Hq/Hk);
    causal row i sees keys 0 .. clamp(Sk - Sq + i + 1, 0, Sk) - 1 and a row
    with no visible key is zero.  fp32 scores, fp64 softmax normalisation
    of the visible keys (the reference's online update is the same sum)."""
    hq, sq, d = q.shape[-3:]
    hk, sk, dv = k.shape[-3], k.shape[-2], v.shape[-1]
    g = hq // hk
    sc = f32(scale) if scale > 0 else f32(1.0 / math.sqrt(d))
    lead = q.shape[:-3]
    qf = q.reshape((-1, hq, sq, d)).astype(f32)
    kf = k.reshape((-1, hk, sk, d)).astype(f32)
    vf = v.reshape((-1, hk, sk, dv)).astype(f32)
    out = np.zeros((qf.shape[0], hq, sq, dv), f32)
    for bi in range(qf.shape[0]):
        for h in range(hq):
            kv = h // g
            s = (qf[bi, h] @ kf[bi, kv].T).astype(f32) * sc
            for i in range(sq):
                n = min(max(sk - sq + i + 1, 0), sk) if causal else sk
                if n == 0:
                    continue
                row = s[i, :n].astype(np.float64)
                p = np.exp(row - row.max())
                out[bi, h, i] = (p @ vf[bi, kv, :n].astype(np.float64) / p.sum()).astype(f32)
    return out.reshape(lead + (hq, sq, dv))


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """llama_graph.cpp:22-28 (swiglu): sigmoid(g) * g * up, three fp32 ops."""
    sig = (f32(1.0) / (f32(1.0) + np.exp(-gate.astype(f32)))).astype(f32)
    return ((sig * gate).astype(f32) * up).astype(f32)


# ------------------------------------------------------------- LLaMA graph

@dataclass
class LlamaConfig:
    """examples/common/llama/llama_config.h:7-24."""
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int = 0
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_seq_len: int = 2048
    tie_word_embeddings: bool = False

    @property
    def kv_heads(self) -> int:
        return self.num_kv_heads if self.num_kv_heads > 0 else self.num_heads

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads


# ------------------------------------------- linears: exact and dense

# How a packed Linear computes (Linear.mode):
#   LINEAR_EXACT  the C oracle's QuantizedMatMul (quantized_matmul.cpp:48-267,
#                 the reference's own arithmetic; the default)
#   LINEAR_DENSE  dequantized weights (quant.cpp:106-123, :177-209) times x
#                 with fp32 BLAS: the same sum in another order, for the
#                 many decode steps of full-size models
LINEAR_EXACT, LINEAR_DENSE = "exact", "dense"


def split_rows_fp16(x: np.ndarray) -> np.ndarray:
    """The HIP MFMA path's staging of A (rows > 4): row r is scaled by 2^x_r
    with max|row| * 2^x_r in [2^14, 2^15) (x_r = 0 for an all-zero row or one
    holding an infinity or NaN) and split into hi = fp16(a * 2^x_r) and
    lo = fp16(a * 2^x_r - hi) (fp16 rounding to nearest even, subnormals
    included); returns (hi + lo) * 2^-x_r in float64, the value the MFMAs
    multiply (22 significant bits of each element)."""
    x = np.ascontiguousarray(x, f32)
    special = ~np.isfinite(x).all(axis=-1)
    amax = np.where(special, f32(0), np.abs(x).max(axis=-1) if x.shape[-1] else f32(0))
    _, e = np.frexp(amax.astype(np.float64))
    xr = np.where(amax > 0, 15 - e, 0).astype(np.int64)
    scaled = np.ldexp(x.astype(np.float64), xr[..., None]).astype(f32)          # exact
    with np.errstate(over="ignore", invalid="ignore"):
        hi = scaled.astype(np.float16)
        rest = scaled - hi.astype(f32)                                          # exact in fp32
        rest = np.where(np.isfinite(rest) & (np.abs(rest) <= 65504), rest, f32(0))
        lo = rest.astype(np.float16)
        total = hi.astype(np.float64) + lo.astype(np.float64)
    return np.ldexp(total, -xr[..., None])


def _oracle_threads() -> int:
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def _qmm_rows_parallel(x2, q, s, k, quant_type, block):
    """Q.qmm over row chunks on several threads (the C call releases the
    GIL).  The reference loop computes every row of an M > 1 product on its
    own, so splitting into chunks of at least two rows changes no bit of the
    result (a one-row call would take the M = 1 streaming path instead)."""
    m = x2.shape[0]
    chunks = min(_oracle_threads(), m // 2)
    if chunks < 2:
        return Q.qmm(x2, q, s, k, quant_type, block)
    from concurrent.futures import ThreadPoolExecutor

    edges = np.linspace(0, m, chunks + 1).astype(int)
    with ThreadPoolExecutor(chunks) as ex:
        parts = list(ex.map(lambda lo_hi: Q.qmm(x2[lo_hi[0]:lo_hi[1]], q, s, k, quant_type, block),
                            zip(edges[:-1], edges[1:])))
    return np.concatenate(parts, axis=0)


@dataclass
class Linear:
    """One linear of the graph: fp32 W [K, N], or packed codes + scales
    (QuantizedMatMul with quant_type / block_size)."""
    w: np.ndarray | None = None
    q: np.ndarray | None = None
    s: np.ndarray | None = None
    k: int = 0
    n: int = 0
    quant_type: int = 0
    block: int = 0
    mode: str = LINEAR_EXACT
    _dense: np.ndarray | None = field(default=None, repr=False)

    def codes(self) -> np.ndarray:
        """Integer codes [K, N] (INT4 nibbles sign-extended, quant.cpp:17-22)."""
        if self.quant_type == Q.QUANT_INT8:
            return self.q.view(np.int8)
        b = self.q.view(np.uint8)
        lo = (b & 0xF).astype(np.int8)
        hi = (b >> 4).astype(np.int8)
        lo = np.where(lo >= 8, lo - 16, lo).astype(np.int8)
        hi = np.where(hi >= 8, hi - 16, hi).astype(np.int8)
        out = np.empty((2 * b.shape[0], b.shape[1]), np.int8)
        out[0::2], out[1::2] = lo, hi
        return out[: self.k]

    def dense(self) -> np.ndarray:
        """fp32 W [K, N]: as given, or dequantized by the pinned oracle."""
        if self.quant_type == Q.QUANT_NONE:
            return self.w
        if self._dense is None:
            if self.quant_type == Q.QUANT_INT8 and self.block > 0:
                # blockwise INT8 (QuantizedMatMulAttrs.block_size > 0, no
                # quant.cpp packer): code * the scale of its K block, exact
                rows = np.repeat(np.asarray(self.s, f32).reshape(-1, self.n), self.block, axis=0)[: self.k]
                self._dense = (self.q.view(np.int8).astype(f32) * rows).astype(f32)
            elif self.quant_type == Q.QUANT_INT8:
                self._dense = Q.dequantize_int8(self.q.view(np.int8), self.s)
            else:
                self._dense = Q.dequantize_int4(self.q.view(np.uint8), self.s, self.k, self.block)
        return self._dense

    def __call__(self, x: np.ndarray) -> np.ndarray:
        """llama_graph.cpp:30-44 (apply_linear): QuantizedMatMul when the
        weight is packed, MatMul otherwise."""
        x2 = np.ascontiguousarray(x.reshape(-1, x.shape[-1]), dtype=f32)
        if self.quant_type == Q.QUANT_NONE:
            y = (x2 @ self.w.astype(f32)).astype(f32)
        elif self.mode == LINEAR_EXACT:
            y = _qmm_rows_parallel(x2, self.q.view(np.int8), self.s, self.k, self.quant_type, self.block)
        else:
            y = (x2 @ self.dense()).astype(f32)
        return y.reshape(x.shape[:-1] + (y.shape[-1],))


@dataclass
class LlamaWeights:
    """examples/common/llama/llama_graph.h:16-34 (ForwardWeights), fp32 [K, N]
    linears (HF weights transposed, Q pre-scaled by 1/sqrt(head_dim) as the
    reference loaders do, tinyllama/model_loader.cpp:195-198)."""
    embed: np.ndarray
    final_norm: np.ndarray
    lm_head: Linear
    attn_norm: list = field(default_factory=list)
    ffn_norm: list = field(default_factory=list)
    wq: list = field(default_factory=list)
    wk: list = field(default_factory=list)
    wv: list = field(default_factory=list)
    wo: list = field(default_factory=list)
    gate: list = field(default_factory=list)
    up: list = field(default_factory=list)
    down: list = field(default_factory=list)


def _lin(w: np.ndarray) -> Linear:
    w = np.ascontiguousarray(w, dtype=f32)
    return Linear(w=w, k=w.shape[0], n=w.shape[1])


def load_toy_llama(tensors: dict, cfg: LlamaConfig) -> LlamaWeights:
    """examples/tinyllama/model_loader.cpp:169-202 and :74-144: HF [out, in]
    weights transposed to [in, out]; q_proj also multiplied by
    1/sqrt(head_dim); lm_head falls back to the embedding when tied."""
    scale_q = f32(1.0) / np.sqrt(f32(cfg.head_dim))
    lm = tensors.get("lm_head.weight", tensors["model.embed_tokens.weight"])
    w = LlamaWeights(embed=np.ascontiguousarray(tensors["model.embed_tokens.weight"], f32),
                     final_norm=np.ascontiguousarray(tensors["model.norm.weight"], f32),
                     lm_head=_lin(lm.T))
    for layer in range(cfg.num_layers):
        p = f"model.layers.{layer}."
        w.attn_norm.append(np.ascontiguousarray(tensors[p + "input_layernorm.weight"], f32))
        w.ffn_norm.append(np.ascontiguousarray(tensors[p + "post_attention_layernorm.weight"], f32))
        w.wq.append(_lin((tensors[p + "self_attn.q_proj.weight"].T * scale_q).astype(f32)))
        w.wk.append(_lin(tensors[p + "self_attn.k_proj.weight"].T))
        w.wv.append(_lin(tensors[p + "self_attn.v_proj.weight"].T))
        w.wo.append(_lin(tensors[p + "self_attn.o_proj.weight"].T))
        w.gate.append(_lin(tensors[p + "mlp.gate_proj.weight"].T))
        w.up.append(_lin(tensors[p + "mlp.up_proj.weight"].T))
        w.down.append(_lin(tensors[p + "mlp.down_proj.weight"].T))
    return w


def quantize_linears(w: LlamaWeights, quant_type: int, block: int = 0) -> LlamaWeights:
    """llama_graph.cpp:336-425 (quantize_forward_weights): every linear and
    the lm_head packed with quant.cpp's scheme (INT8 per column when block is
    0, INT4 blocks of `block`, 32 when 0, src/quant.cpp:74-175); norms and
    the embedding stay fp32."""
    def pack(lin: Linear) -> Linear:
        if quant_type == Q.QUANT_INT8:
            q, s = Q.quantize_int8(lin.w)
            return Linear(q=q, s=s, k=lin.k, n=lin.n, quant_type=quant_type, block=0)
        b = block if block > 0 else 32
        q, s = Q.quantize_int4(lin.w, b)
        return Linear(q=q, s=s, k=lin.k, n=lin.n, quant_type=quant_type, block=b)

    out = LlamaWeights(embed=w.embed, final_norm=w.final_norm, lm_head=pack(w.lm_head),
                       attn_norm=w.attn_norm, ffn_norm=w.ffn_norm)
    for name in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
        setattr(out, name, [pack(lin) for lin in getattr(w, name)])
    return out


def set_linear_mode(w: LlamaWeights, mode: str) -> LlamaWeights:
    """Sets every packed linear of `w` (and the lm_head) to `mode`."""
    for lin in [w.lm_head] + [lin for name in ("wq", "wk", "wv", "wo", "gate", "up", "down")
                              for lin in getattr(w, name)]:
        lin.mode = mode
    return w


def load_packed(tensors: dict, cfg: LlamaConfig, quant_type: int, block: int = 0) -> LlamaWeights:
    """Weights from the pre-packed safetensors layout (`<hf linear name>
    .codes` I8 [K or (K+1)/2, N], `.scales` F32, embedding and norms F32;
    names as the HF checkpoint's, the [in, out] orientation of the graph).
    The codes and scales are taken as they are: the oracle dequantizes
    them, so the comparison measures the kernels, not the packing."""
    def lin(name: str, k: int) -> Linear:
        q = np.ascontiguousarray(tensors[name + ".codes"])
        sc = np.ascontiguousarray(tensors[name + ".scales"], f32)
        n = q.shape[1]
        rows = k if quant_type == Q.QUANT_INT8 else (k + 1) // 2
        if q.shape[0] != rows:
            raise ValueError(f"{name}.codes: {q.shape[0]} rows, expected {rows}")
        return Linear(q=q, s=sc, k=k, n=n, quant_type=quant_type, block=block if quant_type == Q.QUANT_INT4 else 0)

    hid, inter = cfg.hidden_size, cfg.intermediate_size
    w = LlamaWeights(embed=np.ascontiguousarray(tensors["model.embed_tokens.weight"], f32),
                     final_norm=np.ascontiguousarray(tensors["model.norm.weight"], f32),
                     lm_head=lin("lm_head.weight", hid))
    for layer in range(cfg.num_layers):
        p = f"model.layers.{layer}."
        w.attn_norm.append(np.ascontiguousarray(tensors[p + "input_layernorm.weight"], f32))
        w.ffn_norm.append(np.ascontiguousarray(tensors[p + "post_attention_layernorm.weight"], f32))
        for name, hf, k in (("wq", "self_attn.q_proj", hid), ("wk", "self_attn.k_proj", hid),
                            ("wv", "self_attn.v_proj", hid), ("wo", "self_attn.o_proj", hid),
                            ("gate", "mlp.gate_proj", hid), ("up", "mlp.up_proj", hid),
                            ("down", "mlp.down_proj", inter)):
            getattr(w, name).append(lin(p + hf + ".weight", k))
    return w


def _layer(cfg: LlamaConfig, w: LlamaWeights, layer: int, h: np.ndarray, pos0: int, kv: dict | None,
           fused: bool) -> np.ndarray:
    """One decoder layer as llama_graph.cpp:53-158 builds it, for `h`
    [S, hidden] at positions pos0..pos0+S-1.  With kv (decode), the new keys
    and values are appended to kv[layer] (Concat on the sequence axis,
    :296-300) before attention; otherwise (prefill) a causal mask applies."""
    s_len = h.shape[0]
    H, Hk, D = cfg.num_heads, cfg.kv_heads, cfg.head_dim
    hn = rmsnorm(h, w.attn_norm[layer], cfg.rms_norm_eps)
    q = w.wq[layer](hn).reshape(s_len, H, D).transpose(1, 0, 2)
    k = w.wk[layer](hn).reshape(s_len, Hk, D).transpose(1, 0, 2)
    v = w.wv[layer](hn).reshape(s_len, Hk, D).transpose(1, 0, 2)
    cos, sin = rope_cache(s_len, D, cfg.rope_theta, pos0)
    q = rope(np.ascontiguousarray(q), cos, sin)
    k = rope(np.ascontiguousarray(k), cos, sin)
    if kv is not None:
        k_all = concat(kv["k"][layer], k, 1) if kv["k"][layer] is not None else k
        v_all = concat(kv["v"][layer], v, 1) if kv["v"][layer] is not None else np.ascontiguousarray(v)
        kv["k"][layer], kv["v"][layer] = k_all, v_all
        causal_needed = s_len > 1
    else:
        k_all, v_all = k, np.ascontiguousarray(v)
        causal_needed = True
    G = H // Hk
    if fused:
        ctx = attention(q, k_all, v_all, 1.0, True)
    else:
        # llama_graph.cpp:98-106: MatMul(q, k^T) (+ causal mask) -> Softmax -> MatMul.
        ka = repeat_kv(k_all, G, 0) if G > 1 else k_all
        va = repeat_kv(v_all, G, 0) if G > 1 else v_all
        scores = matmul(q, transpose(ka, (0, 2, 1)))
        if causal_needed:
            sk = ka.shape[1]
            allowed = np.arange(sk)[None, :] <= (np.arange(s_len)[:, None] + sk - s_len)
            scores = (scores + np.where(allowed, f32(0), f32(-1e9))[None]).astype(f32)
        ctx = matmul(softmax(scores, -1), va)
    o = w.wo[layer](ctx.transpose(1, 0, 2).reshape(s_len, cfg.hidden_size))
    h = (h + o).astype(f32)
    hn2 = rmsnorm(h, w.ffn_norm[layer], cfg.rms_norm_eps)
    ffn = silu_mul(w.gate[layer](hn2), w.up[layer](hn2))
    return (h + w.down[layer](ffn)).astype(f32)


def prefill(cfg: LlamaConfig, w: LlamaWeights, tokens, last_only: bool = False, fused: bool = False):
    """llama_graph.cpp:162-245 (build_forward_graph_prefill): logits for
    every position ([S, vocab]) or only the last ([1, vocab]), and the
    per-layer K/V ([Hkv, S, D], after RoPE) that seed decoding."""
    tokens = np.asarray(tokens, np.int32)
    h = embedding(w.embed, tokens)
    kv = {"k": [None] * cfg.num_layers, "v": [None] * cfg.num_layers}
    for layer in range(cfg.num_layers):
        h = _layer(cfg, w, layer, h, 0, kv, fused)
    hn = rmsnorm(h, w.final_norm, cfg.rms_norm_eps)
    if last_only:
        hn = hn[-1:]
    return w.lm_head(hn), kv


def decode(cfg: LlamaConfig, w: LlamaWeights, token: int, pos: int, kv: dict, fused: bool = False):
    """llama_graph.cpp:247-330 (build_forward_graph_decode): one token at
    position `pos` attending over the cached K/V plus its own; kv is updated
    in place.  Returns logits [1, vocab]."""
    h = embedding(w.embed, np.asarray([token], np.int32))
    for layer in range(cfg.num_layers):
        h = _layer(cfg, w, layer, h, pos, kv, fused)
    return w.lm_head(rmsnorm(h, w.final_norm, cfg.rms_norm_eps))


def greedy(cfg: LlamaConfig, w: LlamaWeights, prompt, steps: int, fused: bool = False):
    """Prefill, then `steps` decode steps with greedy sampling (first index
    of the maximum, examples/tinyllama/sample.cpp:18-38): returns the
    steps + 1 sampled tokens and the last logits."""
    logits, kv = prefill(cfg, w, prompt, last_only=True, fused=fused)
    pos = len(prompt)
    out = [int(np.argmax(logits[-1]))]
    for _ in range(steps):
        logits = decode(cfg, w, out[-1], pos, kv, fused)
        pos += 1
        out.append(int(np.argmax(logits[-1])))
    return out, logits
