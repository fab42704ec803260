"""The LLaMA-graph operators of libvmhip (include/vm_hip.h, "the rest of the
LLaMA graph") against the oracle (oracle/llama_oracle.py) through the C ABI.

Layout operators (embedding, transpose, slice, concat, repeat_kv) move
bytes and must be bit-exact.  Arithmetic operators are fp32 on both sides
with different summation orders and the device's own exp/sqrt, so they
are held to a relative bound written per test (1e-5 of the output's
largest magnitude, 1e-4 where a long dot product or exp chain feeds it).
"""
from __future__ import annotations

import numpy as np
import pytest

import llama_oracle as L

pytestmark = pytest.mark.gpu


def _close(out, ref, rel):
    ref = np.asarray(ref, np.float64)
    err = np.abs(out.astype(np.float64) - ref).max() if ref.size else 0.0
    bound = rel * max(np.abs(ref).max() if ref.size else 0.0, 1e-30)
    assert err <= bound, f"max abs err {err:.3e} > {bound:.3e}"


def test_embedding(hip):
    rng = np.random.default_rng(0)
    table = rng.standard_normal((300, 72)).astype(np.float32)
    for idx in (np.array([5], np.int32), rng.integers(0, 300, (3, 7), dtype=np.int32), np.array([299, 0], np.int32)):
        print("case embedding", idx.shape, flush=True)
        assert np.array_equal(hip.run_embedding(table, idx), L.embedding(table, idx))


@pytest.mark.parametrize("rows,dim", [(1, 64), (5, 2048), (3, 960), (7, 37)])
def test_rmsnorm(hip, rows, dim):
    rng = np.random.default_rng(rows * dim)
    x = rng.standard_normal((rows, dim)).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    print(f"case rmsnorm rows={rows} dim={dim}", flush=True)
    _close(hip.run_rmsnorm(x, w, 1e-5), L.rmsnorm(x, w, 1e-5), 1e-5)


@pytest.mark.parametrize("shape,cache_rows,pos0", [((32, 1, 64), 1, 17), ((4, 9, 64), 9, 0), ((2, 3, 5, 16), 5, 2)])
def test_rope(hip, shape, cache_rows, pos0):
    rng = np.random.default_rng(len(shape) + cache_rows)
    x = rng.standard_normal(shape).astype(np.float32)
    cos, sin = L.rope_cache(cache_rows, shape[-1], 10000.0, pos0)
    print(f"case rope shape={shape} cache_rows={cache_rows}", flush=True)
    _close(hip.run_rope(x, cos, sin), L.rope(x, cos, sin), 1e-6)


@pytest.mark.parametrize("shape,perm", [((5, 32, 64), (1, 0, 2)), ((4, 9, 16), (0, 2, 1)), ((2, 3, 4, 5), None),
                                        ((7,), None), ((2, 1, 3, 1, 4, 2), (5, 3, 1, 0, 2, 4))])
def test_transpose(hip, shape, perm):
    x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    print(f"case transpose shape={shape} perm={perm}", flush=True)
    assert np.array_equal(hip.run_transpose(x, perm), L.transpose(x, perm))


def test_slice(hip):
    x = np.random.default_rng(3).standard_normal((6, 7, 8)).astype(np.float32)
    # (begins, ends, strides) as the graph passes them; the host clamps as the signature does.
    for begins, ends, strides in (([5], [6], [1]), ([1, 2, 0], [6, 7, 8], [2, 3, 1]), ([-2, 0], [100, 3], [])):
        ref = L.slice_(x, begins, ends, strides)
        b, st = [], []
        for ax, dim in enumerate(x.shape):
            if ax < len(begins):
                bb = begins[ax] + dim if begins[ax] < 0 else begins[ax]
                b.append(min(max(bb, 0), dim))
                st.append(strides[ax] if ax < len(strides) and strides[ax] > 0 else 1)
            else:
                b.append(0)
                st.append(1)
        print(f"case slice {begins} {ends} {strides}", flush=True)
        assert np.array_equal(hip.run_slice(x, b, st, ref.shape), ref)


@pytest.mark.parametrize("sa,sb,axis", [((4, 10, 64), (4, 1, 64), 1), ((3, 5), (2, 5), 0), ((2, 3, 4), (2, 3, 1), 2)])
def test_concat(hip, sa, sb, axis):
    rng = np.random.default_rng(4)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    print(f"case concat {sa} {sb} axis={axis}", flush=True)
    assert np.array_equal(hip.run_concat(a, b, axis), L.concat(a, b, axis))


@pytest.mark.parametrize("shape,rep,axis", [((4, 11, 64), 8, 0), ((5, 3, 64), 3, 0), ((2, 4, 6), 2, 1)])
def test_repeat_kv(hip, shape, rep, axis):
    x = np.random.default_rng(5).standard_normal(shape).astype(np.float32)
    print(f"case repeat_kv {shape} x{rep} axis={axis}", flush=True)
    assert np.array_equal(hip.run_repeat_kv(x, rep, axis), L.repeat_kv(x, rep, axis))


def test_elementwise(hip):
    rng = np.random.default_rng(6)
    a = rng.standard_normal(5633).astype(np.float32) * 4
    b = rng.standard_normal(5633).astype(np.float32)
    print("case elementwise", flush=True)
    assert np.array_equal(hip.run_elementwise(hip.EW_ADD, a, b), a + b)
    assert np.array_equal(hip.run_elementwise(hip.EW_MUL, a, b), a * b)
    sig = (np.float32(1) / (np.float32(1) + np.exp(-a))).astype(np.float32)
    _close(hip.run_elementwise(hip.EW_SIGMOID, a), sig, 1e-6)


@pytest.mark.parametrize("shape,axis", [((32, 9, 9), -1), ((4, 700), -1), ((3, 5, 7), 1), ((6, 2), 0)])
def test_softmax(hip, shape, axis):
    x = np.random.default_rng(7).standard_normal(shape).astype(np.float32) * 3
    print(f"case softmax {shape} axis={axis}", flush=True)
    _close(hip.run_softmax(x, axis), L.softmax(x, axis), 1e-5)


@pytest.mark.parametrize("a_shape,b_shape", [((32, 9, 64), (32, 64, 9)), ((32, 9, 9), (32, 9, 64)),
                                             ((3, 70, 33), (3, 33, 130)), ((1, 1, 5), (1, 5, 1))])
def test_matmul(hip, a_shape, b_shape):
    rng = np.random.default_rng(8)
    a = rng.standard_normal(a_shape).astype(np.float32)
    b = rng.standard_normal(b_shape).astype(np.float32)
    print(f"case matmul {a_shape} x {b_shape}", flush=True)
    _close(hip.run_matmul(a, b), L.matmul(a, b), 1e-5)


@pytest.mark.parametrize("hq,hk,sq,sk,d,dv,scale,causal", [
    (32, 4, 1, 37, 64, 64, 1.0, True),      # TinyLlama decode step, GQA 8
    (32, 32, 1, 300, 64, 64, 1.0, True),    # after RepeatKV
    (15, 5, 1, 129, 64, 64, 0.0, True),     # SmolLM2 heads, default scale
    (4, 4, 9, 9, 16, 16, 1.0, True),        # causal prefill
    (8, 2, 5, 12, 32, 24, 0.3, True),       # Sk > Sq, Dv != D
    (4, 2, 6, 6, 16, 16, 0.0, False),       # non-causal
])
def test_attention(hip, hq, hk, sq, sk, d, dv, scale, causal):
    rng = np.random.default_rng(hq * 100 + sk)
    q = rng.standard_normal((2, hq, sq, d)).astype(np.float32) * 0.5
    k = rng.standard_normal((2, hk, sk, d)).astype(np.float32) * 0.5
    v = rng.standard_normal((2, hk, sk, dv)).astype(np.float32)
    print(f"case attention hq={hq} hk={hk} sq={sq} sk={sk} d={d} dv={dv} causal={causal}", flush=True)
    _close(hip.run_attention(q, k, v, scale, causal), L.attention(q, k, v, scale, causal), 1e-5)


@pytest.mark.parametrize("hq,hk,sk,d,dv", [
    (15, 5, 129, 64, 64),    # SmolLM2 decode, V copied into LDS
    (32, 4, 256, 64, 64),    # TinyLlama heads, V in LDS
    (32, 4, 700, 64, 64),    # V read from global memory (does not fit LDS)
    (8, 2, 5, 32, 24),       # Dv != D
    (4, 2, 33, 18, 18),      # D not a multiple of 4 (scalar loads, V from global)
])
def test_attention_single_row_kernel_matches_the_row_kernel(hip, hq, hk, sk, d, dv):
    """Sq = 1 runs attention_row_kernel (four waves per row); the same row
    inside a two-row non-causal call runs attention_kernel.  Both follow one
    fp32 operation order, so the outputs agree bit for bit."""
    rng = np.random.default_rng(hq * 7 + sk)
    q = rng.standard_normal((2, hq, 1, d)).astype(np.float32) * 0.5
    k = rng.standard_normal((2, hk, sk, d)).astype(np.float32) * 0.5
    v = rng.standard_normal((2, hk, sk, dv)).astype(np.float32)
    print(f"case attention row hq={hq} hk={hk} sk={sk} d={d} dv={dv}", flush=True)
    one = hip.run_attention(q, k, v, 0.0, True)
    two = hip.run_attention(np.concatenate([q, q], axis=2), k, v, 0.0, False)
    assert one.tobytes() == np.ascontiguousarray(two[:, :, :1, :]).tobytes()
