"""The resident decoder's kernels (include/vm_hip.h: add_rmsnorm, silu_mul,
argmax, rope_kv_append, attention_decode, attention_prefill) against the
oracle (oracle/llama_oracle.py) through the C ABI.

Bounds: the residual add is one fp32 addition on both sides, so h must be
bit-exact; the norm, SwiGLU and attention are fp32 with a different
summation order and the device's own exp/sqrt, held to 1e-5 of the
output's largest magnitude; argmax and the cache writes of rope_kv_append
are exact (indices, copies).
"""
from __future__ import annotations


import numpy as np
import pytest

import llama_oracle as L

pytestmark = pytest.mark.gpu


def _close(out, ref, rel, what=""):
    ref = np.asarray(ref, np.float64)
    err = np.abs(np.asarray(out, np.float64) - ref).max()
    bound = rel * max(np.abs(ref).max(), 1e-30)
    assert err <= bound, f"{what}: max abs err {err:.3e} > {bound:.3e}"


def _lib(hip):
    return hip.open_library()


def _dev(hip, a, dtype=np.float32):
    return hip.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype))


@pytest.mark.parametrize("rows,dim", [(1, 2048), (3, 960), (2, 64), (1, 4100), (2, 8192), (1, 37), (1, 10000)])
@pytest.mark.parametrize("with_delta", [False, True])
def test_add_rmsnorm(hip, rows, dim, with_delta):
    rng = np.random.default_rng(rows * 7 + dim)
    h = (rng.standard_normal((rows, dim)) * 2).astype(np.float32)
    d = rng.standard_normal((rows, dim)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    dh, dd, dw, dn = _dev(hip, h), _dev(hip, d), _dev(hip, w), hip.DeviceBuffer(rows * dim * 4)
    print(f"case add_rmsnorm rows={rows} dim={dim} delta={with_delta}", flush=True)
    hip.check(_lib(hip).vm_hip_add_rmsnorm_f32(dh.ptr, dd.ptr if with_delta else None, dw.ptr, dn.ptr, rows, dim,
                                               1e-5, None))
    h_ref = (h + d).astype(np.float32) if with_delta else h
    assert np.array_equal(dh.download(np.float32, (rows, dim)), h_ref)
    _close(dn.download(np.float32, (rows, dim)), L.rmsnorm(h_ref, w, 1e-5), 1e-5, "rmsnorm")


def test_add_rmsnorm_unaligned_rows_take_the_generic_path(hip):
    rng = np.random.default_rng(3)
    dim = 2048
    h = rng.standard_normal(dim + 1).astype(np.float32)
    w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    dh, dw, dn = _dev(hip, h), _dev(hip, w), hip.DeviceBuffer((dim + 1) * 4)
    # rows start one float into the buffers: not 16-byte aligned
    hip.check(_lib(hip).vm_hip_add_rmsnorm_f32(dh.addr + 4, None, dw.ptr, dn.addr + 4, 1, dim, 1e-5, None))
    _close(dn.download(np.float32, (dim + 1,))[1:], L.rmsnorm(h[1:], w, 1e-5), 1e-5, "rmsnorm")


@pytest.mark.parametrize("rows,inter", [(1, 5632), (5, 2560), (3, 37), (2, 6)])
def test_silu_mul(hip, rows, inter):
    rng = np.random.default_rng(rows + inter)
    gu = (rng.standard_normal((rows, 2 * inter)) * 3).astype(np.float32)
    dg, do = _dev(hip, gu), hip.DeviceBuffer(rows * inter * 4)
    print(f"case silu_mul rows={rows} inter={inter}", flush=True)
    hip.check(_lib(hip).vm_hip_silu_mul_f32(dg.ptr, do.ptr, rows, inter, None))
    _close(do.download(np.float32, (rows, inter)), L.silu_mul(gu[:, :inter], gu[:, inter:]), 1e-5, "silu_mul")


def _argmax_ref(x):
    best, idx = None, -1
    for i, v in enumerate(x.tolist()):
        if v != v:
            continue
        if idx < 0 or v > best:
            best, idx = v, i
    return idx


def _run_argmax(hip, x, offset_floats=0, pos=None, max_seq=0):
    buf = np.concatenate([np.zeros(offset_floats, np.float32), x]).astype(np.float32)
    dx, dt = _dev(hip, buf), hip.DeviceBuffer(4)
    dpos = dseq = None
    if pos is not None:
        dpos = _dev(hip, np.array([pos], np.int32), np.int32)
        dseq = _dev(hip, np.full(max_seq, -7, np.int32), np.int32)
    hip.check(_lib(hip).vm_hip_argmax_f32(dx.addr + 4 * offset_floats, x.size, dt.ptr, dpos.ptr if dpos else None,
                                          dseq.ptr if dseq else None, max_seq, None))
    tok = int(dt.download(np.int32, (1,))[0])
    if pos is None:
        return tok
    return tok, int(dpos.download(np.int32, (1,))[0]), dseq.download(np.int32, (max_seq,))


@pytest.mark.parametrize("n", [1, 5, 32000, 49152, 70001])
def test_argmax(hip, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    print(f"case argmax n={n}", flush=True)
    assert _run_argmax(hip, x) == _argmax_ref(x)
    # ties resolve to the first index; NaN is skipped
    if n >= 5:
        x[n // 3] = x[n - 1] = 50.0
        x[n // 2] = np.nan
        x[0] = np.nan
        assert _run_argmax(hip, x) == _argmax_ref(x) == n // 3
        assert _run_argmax(hip, x, offset_floats=1) == n // 3      # unaligned: scalar path


def test_argmax_advances_position_and_records_token(hip):
    x = np.zeros(1000, np.float32)
    x[417] = 3.0
    tok, pos, seq = _run_argmax(hip, x, pos=9, max_seq=16)
    assert (tok, pos) == (417, 10)
    assert seq[10] == 417 and np.all(np.delete(seq, 10) == -7)
    # at the end of the buffer the token is not stored, the position still advances
    tok, pos, seq = _run_argmax(hip, x, pos=15, max_seq=16)
    assert (tok, pos) == (417, 16) and np.all(seq == -7)


def _attention_case(hip, heads, kv_heads, d, max_seq, p, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((heads, d)).astype(np.float32)
    kc = rng.standard_normal((kv_heads, max_seq, d)).astype(np.float32)
    vc = rng.standard_normal((kv_heads, max_seq, d)).astype(np.float32)
    dq, dk, dv = _dev(hip, q), _dev(hip, kc), _dev(hip, vc)
    dpos, do = _dev(hip, np.array([p], np.int32), np.int32), hip.DeviceBuffer(heads * d * 4)
    scale = 1.0 / np.sqrt(d)
    hip.check(_lib(hip).vm_hip_attention_decode_f32(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, do.ptr, heads, kv_heads, d,
                                                    max_seq, scale, None))
    n = min(p + 1, max_seq)
    ref = L.attention(q[:, None, :], kc[:, :n], vc[:, :n], scale, causal=False)[:, 0]
    return do.download(np.float32, (heads, d)), ref


@pytest.mark.parametrize("heads,kv_heads,d,max_seq,positions", [
    (32, 4, 64, 776, [0, 62, 63, 64, 511, 767, 775]),   # TinyLlama: G = 8
    (15, 5, 64, 264, [0, 127, 200, 263]),                # SmolLM2-360M: G = 3
    (16, 1, 64, 300, [5, 130, 299]),                     # G = 16 (the maximum)
    (8, 8, 128, 100, [0, 31, 32, 99]),                   # head_dim 128, G = 1
    (8, 2, 128, 1100, [1099]),                           # 35 chunks: three merge batches
])
def test_attention_decode(hip, heads, kv_heads, d, max_seq, positions):
    for i, p in enumerate(positions):
        print(f"case attention_decode H={heads} Hkv={kv_heads} D={d} max_seq={max_seq} pos={p}", flush=True)
        out, ref = _attention_case(hip, heads, kv_heads, d, max_seq, p, seed=100 * i + heads)
        _close(out, ref, 1e-5, f"pos {p}")


def test_attention_decode_repeated_calls_reset_tickets(hip):
    # The chunk tickets live in the per-stream workspace and are reset by the
    # merging workgroup: calls with different chunk counts in a row agree.
    for p in (700, 3, 390, 700):
        out, ref = _attention_case(hip, 32, 4, 64, 776, p, seed=7)
        _close(out, ref, 1e-5, f"pos {p}")


def test_rope_kv_append(hip):
    heads, kv_heads, d, max_seq, rows, p0 = 8, 2, 64, 40, 3, 5
    rng = np.random.default_rng(11)
    width = (heads + 2 * kv_heads) * d
    qkv = rng.standard_normal((rows, width)).astype(np.float32)
    cos, sin = L.rope_cache(max_seq, d, 10000.0)
    kc0 = rng.standard_normal((kv_heads, max_seq, d)).astype(np.float32)
    vc0 = rng.standard_normal((kv_heads, max_seq, d)).astype(np.float32)
    dqkv, dc, ds = _dev(hip, qkv), _dev(hip, cos), _dev(hip, sin)
    dk, dv, dq = _dev(hip, kc0), _dev(hip, vc0), hip.DeviceBuffer(heads * rows * d * 4)
    dpos = _dev(hip, np.array([p0], np.int32), np.int32)
    hip.check(_lib(hip).vm_hip_rope_kv_append_f32(dqkv.ptr, rows, dc.ptr, ds.ptr, dpos.ptr, dq.ptr, dk.ptr, dv.ptr,
                                                  heads, kv_heads, d, max_seq, None))
    qs = qkv[:, :heads * d].reshape(rows, heads, d).transpose(1, 0, 2)
    ks = qkv[:, heads * d:(heads + kv_heads) * d].reshape(rows, kv_heads, d).transpose(1, 0, 2)
    vs = qkv[:, (heads + kv_heads) * d:].reshape(rows, kv_heads, d).transpose(1, 0, 2)
    c, s = cos[p0:p0 + rows], sin[p0:p0 + rows]
    _close(dq.download(np.float32, (heads, rows, d)), L.rope(np.ascontiguousarray(qs), c, s), 1e-6, "q")
    kc, vc = kc0.copy(), vc0.copy()
    kc[:, p0:p0 + rows] = L.rope(np.ascontiguousarray(ks), c, s)
    vc[:, p0:p0 + rows] = vs
    _close(dk.download(np.float32, kc.shape), kc, 1e-6, "k cache")
    assert np.array_equal(dv.download(np.float32, vc.shape), vc)


# (512, 0, ...) is TinyLlama's 512-token prefill (eight 64-key tiles for the
# last query rows); (256, 300, ...) continues a cached prefix.  Grids of at
# most 512 64-row tiles split each workgroup's keys over two wave pairs;
# (600, 0, 64, ...) has 640 tiles and runs the one-group form.
@pytest.mark.parametrize("rows,p0,heads,kv_heads,max_seq", [(19, 0, 8, 2, 96), (64, 0, 8, 2, 96), (70, 10, 8, 2, 96),
                                                        (200, 0, 32, 4, 256), (130, 77, 15, 5, 256),
                                                        (1, 40, 8, 8, 64), (512, 0, 32, 4, 768),
                                                        (256, 300, 16, 4, 768), (33, 0, 4, 1, 40),
                                                        (600, 0, 64, 8, 640), (600, 30, 64, 8, 640)])
def test_attention_prefill(hip, rows, p0, heads, kv_heads, max_seq):
    d = 64
    rng = np.random.default_rng(rows + p0)
    q = rng.standard_normal((heads, rows, d)).astype(np.float32)
    kc = rng.standard_normal((kv_heads, max_seq, d)).astype(np.float32)
    vc = rng.standard_normal((kv_heads, max_seq, d)).astype(np.float32)
    dq, dk, dv = _dev(hip, q), _dev(hip, kc), _dev(hip, vc)
    dpos, do = _dev(hip, np.array([p0], np.int32), np.int32), hip.DeviceBuffer(rows * heads * d * 4)
    scale = 0.125
    hip.check(_lib(hip).vm_hip_attention_prefill_f32(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, do.ptr, rows, heads, kv_heads,
                                                     d, max_seq, scale, None))
    n = p0 + rows
    ref = L.attention(q, kc[:, :n], vc[:, :n], scale, causal=True)   # [H, rows, D]
    _close(do.download(np.float32, (rows, heads, d)), ref.transpose(1, 0, 2), 1e-5, "prefill")


def test_decode_ops_reject_bad_arguments(hip):
    lib = _lib(hip)
    buf = hip.DeviceBuffer(1 << 16)
    assert lib.vm_hip_attention_decode_f32(buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 32, 4, 96, 64, 0.0,
                                           None) == hip.EUNSUPPORTED
    assert lib.vm_hip_attention_decode_f32(buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 34, 2, 64, 64, 0.0,
                                           None) == hip.EINVAL     # 17 query heads per KV head
    assert lib.vm_hip_attention_decode_f32(buf.addr + 4, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 8, 2, 64, 64, 0.0,
                                           None) == hip.EINVAL     # unaligned q
    assert lib.vm_hip_argmax_f32(buf.ptr, 0, buf.ptr, None, None, 0, None) == hip.EINVAL
    assert lib.vm_hip_add_rmsnorm_f32(None, None, buf.ptr, buf.ptr, 1, 8, 1e-5, None) == hip.EINVAL
    assert "null" in hip.last_error()
