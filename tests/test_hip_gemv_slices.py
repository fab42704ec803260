"""Split-K decode GEMV with consumer-side reduction
(vm_hip_qmm_gemv_slices_f32) and the kernels that consume its partial
slices (add_rmsnorm_slices, rope_kv_append_slices, argmax_slices,
slices_sum), against the oracle through the C ABI.

The sum of the slices must equal the reference QuantizedMatMul
(src/cpu/ops/quantized_matmul.cpp:48-141) within 1e-5 of max|ref|: fp32
accumulation on both sides, only the summation order differs, and a wrong
nibble, scale index, block or slice would miss the bound by orders of
magnitude.  Argmax results and copied values are exact.
"""
from __future__ import annotations

import numpy as np
import pytest

import llama_oracle as L
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _normal(shape, seed, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def _close(out, ref, rel, what=""):
    ref = np.asarray(ref, np.float64)
    err = np.abs(np.asarray(out, np.float64) - ref).max()
    bound = rel * max(np.abs(ref).max(), 1e-30)
    assert err <= bound, f"{what}: max abs err {err:.3e} > {bound:.3e}"


def _dev(hip, a, dtype=np.float32):
    return hip.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype))


def _pack(k, n, qt, block, seed):
    w = _normal((k, n), seed, 0.02)
    if qt == O.QUANT_INT4:
        p, s = O.quantize_int4(w, block)
        return p.view(np.int8), s
    if block:
        # INT8 blockwise scales, the reference's blocked INT8 path
        # (quantized_matmul.cpp:97-122): per (block, column) max / 127.
        nb = (k + block - 1) // block
        s = np.ones((nb, n), np.float32)
        q = np.zeros((k, n), np.int8)
        for b in range(nb):
            blk = w[b * block:(b + 1) * block]
            mx = np.abs(blk).max(axis=0)
            sc = np.where(mx > 0, mx / np.float32(127.0), np.float32(1.0)).astype(np.float32)
            s[b] = sc
            q[b * block:(b + 1) * block] = np.clip(np.round(blk / sc), -127, 127).astype(np.int8)
        return q, s
    return O.quantize_int8(w)


def _count(hip, k, n, qt, block, max_slices):
    import ctypes
    out = ctypes.c_int(0)
    hip.check(hip.open_library().vm_hip_gemv_slices_count(k, n, qt, block, max_slices, ctypes.byref(out)))
    return out.value


def _run(hip, x_src, kind, act_slices, q, s, k, n, qt, block, max_slices=64):
    lib = hip.open_library()
    sl = _count(hip, k, n, qt, block, max_slices)
    assert 1 <= sl <= max_slices
    dx, dq, ds, do = _dev(hip, x_src), _dev(hip, q, np.int8), _dev(hip, s), hip.DeviceBuffer(sl * n * 4)
    hip.check(lib.vm_hip_qmm_gemv_slices_f32(dx.ptr, kind, act_slices, dq.ptr, ds.ptr, do.ptr, k, n, qt, block,
                                             max_slices, None))
    return do.download(np.float32, (sl, n)), sl


CASES = [
    # (k, n, quant, block, max_slices): TinyLlama INT4 decode shapes, SmolLM2 INT8, tails
    (2048, 2560, O.QUANT_INT4, 32, 64),
    (2048, 2048, O.QUANT_INT4, 32, 64),
    (5632, 2048, O.QUANT_INT4, 32, 22),
    (2048, 11264, O.QUANT_INT4, 32, 64),
    (2048, 32000, O.QUANT_INT4, 32, 8),
    (960, 1600, O.QUANT_INT4, 32, 64),      # partial last tile, K not a multiple of a workgroup's rows
    (64, 16, O.QUANT_INT4, 32, 64),
    (2048, 2048, O.QUANT_INT4, 64, 64),
    (960, 1600, O.QUANT_INT8, 0, 64),       # SmolLM2-360M q|k|v
    (2560, 960, O.QUANT_INT8, 0, 22),       # SmolLM2-360M down
    (960, 49152, O.QUANT_INT8, 0, 8),       # SmolLM2-360M lm_head
    (1024, 512, O.QUANT_INT8, 32, 64),      # INT8 blockwise
]


@pytest.mark.parametrize("k,n,qt,block,max_slices", CASES)
def test_gemv_slices_plain(hip, k, n, qt, block, max_slices):
    q, s = _pack(k, n, qt, block, k * 7 + n)
    x = _normal((1, k), k + n)
    print(f"case gemv_slices plain k={k} n={n} qt={qt} block={block}", flush=True)
    out, sl = _run(hip, x, hip.GEMV_SRC_PLAIN, 0, q, s, k, n, qt, block, max_slices)
    ref = O.qmm(x, q, s, k, qt, block)
    _close(out.sum(axis=0, dtype=np.float64), ref[0], TOL, f"{sl} slices")


@pytest.mark.parametrize("in_slices", [1, 3, 16, 22])
def test_gemv_slices_from_slices(hip, in_slices):
    k, n = 2048, 2048
    q, s = _pack(k, n, O.QUANT_INT4, 32, 5)
    src = _normal((in_slices, k), in_slices)
    x = src[0].copy()
    for i in range(1, in_slices):
        x = (x + src[i]).astype(np.float32)
    print(f"case gemv_slices from {in_slices} slices", flush=True)
    out, _ = _run(hip, src, hip.GEMV_SRC_SLICES, in_slices, q, s, k, n, O.QUANT_INT4, 32)
    _close(out.sum(axis=0, dtype=np.float64), O.qmm(x[None], q, s, k, O.QUANT_INT4, 32)[0], TOL)


@pytest.mark.parametrize("k,n,qt,block,in_slices", [(5632, 2048, O.QUANT_INT4, 32, 16),
                                                     (2560, 960, O.QUANT_INT8, 0, 15),
                                                     (256, 64, O.QUANT_INT4, 32, 1)])
def test_gemv_slices_swiglu(hip, k, n, qt, block, in_slices):
    q, s = _pack(k, n, qt, block, 9)
    gu = _normal((in_slices, 2 * k), k, 0.7)
    g, u = gu[0, :k].copy(), gu[0, k:].copy()
    for i in range(1, in_slices):
        g = (g + gu[i, :k]).astype(np.float32)
        u = (u + gu[i, k:]).astype(np.float32)
    x = L.silu_mul(g, u)
    print(f"case gemv_slices swiglu k={k} n={n} in_slices={in_slices}", flush=True)
    out, _ = _run(hip, gu, hip.GEMV_SRC_SWIGLU, in_slices, q, s, k, n, qt, block, 22)
    _close(out.sum(axis=0, dtype=np.float64), O.qmm(x[None], q, s, k, qt, block)[0], TOL)


def test_gemv_slices_is_deterministic_and_counts_are_stable(hip):
    k, n = 5632, 2048
    q, s = _pack(k, n, O.QUANT_INT4, 32, 1)
    x = _normal((1, k), 2)
    a, sa = _run(hip, x, hip.GEMV_SRC_PLAIN, 0, q, s, k, n, O.QUANT_INT4, 32, 22)
    b, sb = _run(hip, x, hip.GEMV_SRC_PLAIN, 0, q, s, k, n, O.QUANT_INT4, 32, 22)
    assert sa == sb == _count(hip, k, n, O.QUANT_INT4, 32, 22)
    assert np.array_equal(a, b)
    # a tighter slice limit gives fewer slices, same result within fp32 rounding
    c, sc = _run(hip, x, hip.GEMV_SRC_PLAIN, 0, q, s, k, n, O.QUANT_INT4, 32, 11)
    assert sc <= 11
    _close(c.sum(axis=0, dtype=np.float64), a.sum(axis=0, dtype=np.float64), TOL)


def test_gemv_slices_rejects_unsupported(hip):
    import ctypes
    lib = hip.open_library()
    out = ctypes.c_int(0)
    assert lib.vm_hip_gemv_slices_count(2048, 100, O.QUANT_INT4, 32, 64, ctypes.byref(out)) == hip.EINVAL
    assert lib.vm_hip_gemv_slices_count(2048, 2048, O.QUANT_INT8, 8, 64, ctypes.byref(out)) == hip.EUNSUPPORTED
    assert lib.vm_hip_gemv_slices_count(5632, 2048, O.QUANT_INT4, 32, 2, ctypes.byref(out)) == hip.EUNSUPPORTED
    buf = hip.DeviceBuffer(1 << 20)
    assert lib.vm_hip_qmm_gemv_slices_f32(buf.addr + 4, hip.GEMV_SRC_PLAIN, 0, buf.ptr, buf.ptr, buf.ptr, 256, 64,
                                          O.QUANT_INT4, 32, 64, None) == hip.EINVAL      # unaligned activation


@pytest.mark.parametrize("dim,slices", [(2048, 0), (2048, 1), (2048, 16), (960, 22), (5632, 4), (8192, 3)])
def test_add_rmsnorm_slices(hip, dim, slices):
    h = _normal(dim, dim, 2.0)
    d = _normal((max(slices, 1), dim), slices + 1)
    w = np.random.default_rng(3).uniform(0.5, 1.5, dim).astype(np.float32)
    dh, dd, dw, dn = _dev(hip, h), _dev(hip, d), _dev(hip, w), hip.DeviceBuffer(dim * 4)
    print(f"case add_rmsnorm_slices dim={dim} slices={slices}", flush=True)
    hip.check(hip.open_library().vm_hip_add_rmsnorm_slices_f32(dh.ptr, dd.ptr if slices else None, slices, dw.ptr,
                                                               dn.ptr, dim, 1e-5, None))
    ref_h = h.copy()
    for i in range(slices):
        ref_h = (ref_h + d[i]).astype(np.float32)
    assert np.array_equal(dh.download(np.float32, (dim,)), ref_h)   # same additions in the same order
    _close(dn.download(np.float32, (dim,)), L.rmsnorm(ref_h, w, 1e-5), 1e-5, "rmsnorm")


def test_rope_kv_append_slices(hip):
    heads, kv_heads, d, max_seq, p0, slices = 8, 2, 64, 40, 17, 5
    width = (heads + 2 * kv_heads) * d
    qkv = _normal((slices, width), 4)
    tot = qkv[0].copy()
    for i in range(1, slices):
        tot = (tot + qkv[i]).astype(np.float32)
    cos, sin = L.rope_cache(max_seq, d, 10000.0)
    kc0, vc0 = _normal((kv_heads, max_seq, d), 5), _normal((kv_heads, max_seq, d), 6)
    dq, dc, ds = _dev(hip, qkv), _dev(hip, cos), _dev(hip, sin)
    dk, dv, dqo = _dev(hip, kc0), _dev(hip, vc0), hip.DeviceBuffer(heads * d * 4)
    dpos = _dev(hip, np.array([p0], np.int32), np.int32)
    hip.check(hip.open_library().vm_hip_rope_kv_append_slices_f32(dq.ptr, slices, dc.ptr, ds.ptr, dpos.ptr, dqo.ptr,
                                                                  dk.ptr, dv.ptr, heads, kv_heads, d, max_seq, None))
    c, s = cos[p0:p0 + 1], sin[p0:p0 + 1]
    qs = tot[:heads * d].reshape(heads, 1, d)
    ks = tot[heads * d:(heads + kv_heads) * d].reshape(kv_heads, 1, d)
    vs = tot[(heads + kv_heads) * d:].reshape(kv_heads, d)
    _close(dqo.download(np.float32, (heads, 1, d)), L.rope(qs, c, s), 1e-6, "q")
    kc, vc = kc0.copy(), vc0.copy()
    kc[:, p0] = L.rope(ks, c, s)[:, 0]
    vc[:, p0] = vs
    _close(dk.download(np.float32, kc.shape), kc, 1e-6, "k cache")
    assert np.array_equal(dv.download(np.float32, vc.shape), vc)


@pytest.mark.parametrize("n,slices", [(32000, 8), (49152, 4), (1000, 3), (37, 2)])
def test_argmax_and_sum_of_slices(hip, n, slices):
    x = _normal((slices, n), n)
    tot = x[0].copy()
    for i in range(1, slices):
        tot = (tot + x[i]).astype(np.float32)
    dx, dt, ds = _dev(hip, x), hip.DeviceBuffer(4), hip.DeviceBuffer(n * 4)
    lib = hip.open_library()
    hip.check(lib.vm_hip_argmax_slices_f32(dx.ptr, slices, n, dt.ptr, None, None, 0, None))
    hip.check(lib.vm_hip_slices_sum_f32(dx.ptr, slices, n, ds.ptr, None))
    assert np.array_equal(ds.download(np.float32, (n,)), tot)
    assert int(dt.download(np.int32, (1,))[0]) == int(np.argmax(tot))


@pytest.mark.parametrize("n,slices", [(32000, 4), (49152, 4), (1000, 3), (4096, 9), (37, 2), (1028, 1)])
def test_argmax_across_workgroups(hip, n, slices):
    """vm_hip_argmax_slices_ws_f32 (one candidate per 1024 elements, the last
    workgroup reduces): the sum of slices' first maximum, NaN skipped, the
    position advanced and the token recorded; repeated calls reuse the
    workspace (its ticket is reset); ties across workgroups resolve to the
    lowest index."""
    x = _normal((slices, n), n + 3)
    tot = x[0].copy()
    for i in range(1, slices):
        tot = (tot + x[i]).astype(np.float32)
    lib = hip.open_library()
    wsb = lib.vm_hip_argmax_workspace_bytes(n)
    assert wsb >= 256 + 8 * ((n + 1023) // 1024)
    ws = _dev(hip, np.zeros(wsb // 4 + 1, np.float32))
    dx, dt = _dev(hip, x), hip.DeviceBuffer(4)
    dpos = _dev(hip, np.array([3], np.int32), np.int32)
    dseq = _dev(hip, np.full(8, -7, np.int32), np.int32)
    print(f"case argmax_ws n={n} slices={slices}", flush=True)
    for call in range(3):
        hip.check(lib.vm_hip_argmax_slices_ws_f32(dx.ptr, slices, n, dt.ptr, dpos.ptr, dseq.ptr, 8, ws.ptr, wsb, None))
        assert int(dt.download(np.int32, (1,))[0]) == int(np.argmax(tot)), call
    assert int(dpos.download(np.int32, (1,))[0]) == 6
    seq = dseq.download(np.int32, (8,))
    assert list(seq[4:7]) == [int(np.argmax(tot))] * 3 and seq[7] == -7
    if n >= 3000:
        # equal maxima in two workgroups and a NaN: the lower index wins
        y = x.copy()
        y[:, :] = 0.0
        y[0, 2100] = y[0, 1500] = 9.0
        y[0, 5] = np.nan
        dy = _dev(hip, y)
        hip.check(lib.vm_hip_argmax_slices_ws_f32(dy.ptr, slices, n, dt.ptr, None, None, 0, ws.ptr, wsb, None))
        assert int(dt.download(np.int32, (1,))[0]) == 1500
    assert lib.vm_hip_argmax_slices_ws_f32(dx.ptr, slices, n, dt.ptr, None, None, 0, ws.ptr, 16, None) != 0


def _src(hip, **kw):
    s = hip.GemvSrc()
    for key, val in kw.items():
        setattr(s, key, val)
    return s


def _run_src(hip, src, q, s, k, n, qt, block, max_slices=64):
    import ctypes
    sl = _count(hip, k, n, qt, block, max_slices)
    dq, ds, do = _dev(hip, q, np.int8), _dev(hip, s), hip.DeviceBuffer(sl * n * 4)
    hip.check(hip.open_library().vm_hip_qmm_gemv_slices_src_f32(ctypes.byref(src), dq.ptr, ds.ptr, do.ptr, k, n, qt,
                                                                 block, max_slices, None))
    return do.download(np.float32, (sl, n)), sl


@pytest.mark.parametrize("k,n,qt,block,delta_slices", [(2048, 2560, O.QUANT_INT4, 32, 22),
                                                       (2048, 11264, O.QUANT_INT4, 32, 16),
                                                       (960, 1600, O.QUANT_INT8, 0, 20),
                                                       (2048, 2560, O.QUANT_INT4, 32, 0)])
def test_gemv_slices_residual_norm_source(hip, k, n, qt, block, delta_slices):
    """NORMRES: x = (h + sum delta) * w staged per split; the consumer's
    scale 1/rms from the per-split sums of squares completes RMSNorm."""
    q, s = _pack(k, n, qt, block, 21)
    h = _normal(k, 1, 2.0)
    d = _normal((max(delta_slices, 1), k), 2)
    w = np.random.default_rng(4).uniform(0.5, 1.5, k).astype(np.float32)
    sl = _count(hip, k, n, qt, block, 64)
    dh, dd, dw = _dev(hip, h), _dev(hip, d), _dev(hip, w)
    dho, dss = hip.DeviceBuffer(k * 4), hip.DeviceBuffer(sl * 4)
    src = _src(hip, kind=hip.GEMV_SRC_NORMRES, slices=delta_slices, act=dh.addr, delta=dd.addr if delta_slices else None,
               norm_w=dw.addr, h_out=dho.addr, ss_out=dss.addr)
    print(f"case gemv_slices normres k={k} n={n} delta_slices={delta_slices}", flush=True)
    out, _ = _run_src(hip, src, q, s, k, n, qt, block)
    ref_h = h.copy()
    for i in range(delta_slices):
        ref_h = (ref_h + d[i]).astype(np.float32)
    # the slices are added in a fixed grouping of their own (per staging part)
    _close(dho.download(np.float32, (k,)), ref_h, 1e-6, "residual")
    ss = dss.download(np.float32, (sl,)).astype(np.float64)
    assert abs(ss.sum() - (ref_h.astype(np.float64) ** 2).sum()) <= 1e-5 * (ref_h.astype(np.float64) ** 2).sum()
    inv = 1.0 / np.sqrt(ss.sum() / k + 1e-5)
    ref = O.qmm(L.rmsnorm(ref_h, w, 1e-5)[None], q, s, k, qt, block)[0]
    _close(out.sum(axis=0, dtype=np.float64) * inv, ref, TOL, "normed projection")


@pytest.mark.parametrize("heads,kv_heads,d,max_seq,p,slices", [(32, 4, 64, 769, 767, 16),   # TinyLlama, bench's last
                                                                (32, 4, 64, 776, 775, 16),   # last row of the cache
                                                                (15, 5, 64, 257, 255, 15),   # SmolLM2, bench's last
                                                                (32, 4, 64, 584, 530, 16),
                                                                (32, 4, 64, 584, 0, 16),
                                                                (32, 4, 64, 584, 63, 3),
                                                                (15, 5, 64, 264, 200, 15),
                                                                (8, 2, 128, 100, 64, 4)])
def test_attention_decode_slices_and_merge_source(hip, heads, kv_heads, d, max_seq, p, slices):
    """Fused decode attention (slice sums, RMSNorm scale, RoPE, in-place
    K/V append, per-chunk partials) followed by the output projection that
    merges the partials while staging: against the oracle's RMSNorm-scaled
    q/k/v, RoPE, attention and QuantizedMatMul."""
    import ctypes
    lib = hip.open_library()
    width = (heads + 2 * kv_heads) * d
    hidden = heads * d
    qkv = _normal((slices, width), p + 1)
    ss = np.abs(_normal(7, 3, 50.0)) + 1.0
    inv = np.float32(1.0 / np.sqrt(ss.astype(np.float32).sum(dtype=np.float32) / np.float32(hidden) + np.float32(1e-5)))
    cos, sin = L.rope_cache(max_seq, d, 10000.0)
    kc0, vc0 = _normal((kv_heads, max_seq, d), 5), _normal((kv_heads, max_seq, d), 6)
    ch, chs = ctypes.c_int(0), ctypes.c_int(0)
    hip.check(lib.vm_hip_attention_decode_chunks(d, max_seq, ctypes.byref(ch), ctypes.byref(chs)))
    dqkv, dss, dc, dsn = _dev(hip, qkv), _dev(hip, ss), _dev(hip, cos), _dev(hip, sin)
    dk, dv = _dev(hip, kc0), _dev(hip, vc0)
    dpos = _dev(hip, np.array([p], np.int32), np.int32)
    dpart = hip.DeviceBuffer(heads * chs.value * (d + 4) * 4)
    print(f"case attention_decode_slices H={heads} Hkv={kv_heads} D={d} p={p} slices={slices}", flush=True)
    hip.check(lib.vm_hip_attention_decode_slices_f32(dqkv.ptr, slices, dss.ptr, ss.size, float(hidden), 1e-5, dc.ptr,
                                                     dsn.ptr, dpos.ptr, dk.ptr, dv.ptr, dpart.ptr, heads, kv_heads, d,
                                                     max_seq, 1.0, None))
    tot = qkv[0].copy()
    for i in range(1, slices):
        tot = (tot + qkv[i]).astype(np.float32)
    tot = (tot * inv).astype(np.float32)
    c, s_ = cos[p:p + 1], sin[p:p + 1]
    qr = L.rope(tot[:hidden].reshape(heads, 1, d), c, s_)
    kr = L.rope(tot[hidden:hidden + kv_heads * d].reshape(kv_heads, 1, d), c, s_)[:, 0]
    vr = tot[hidden + kv_heads * d:].reshape(kv_heads, d)
    kc, vc = kc0.copy(), vc0.copy()
    kc[:, p], vc[:, p] = kr, vr
    _close(dk.download(np.float32, kc.shape), kc, 1e-5, "k cache")
    _close(dv.download(np.float32, vc.shape), vc, 1e-5, "v cache")
    ctx = L.attention(qr, kc[:, :p + 1], vc[:, :p + 1], 1.0, causal=False)[:, 0].reshape(1, hidden)
    # the output projection merges the partials while staging
    qo, so = _pack(hidden, 256, O.QUANT_INT4, 32, 8)
    src = _src(hip, kind=hip.GEMV_SRC_ATTN, act=dpart.addr, pos=dpos.addr, head_dim=d, chunk=ch.value,
               chunks=chs.value, max_seq=max_seq)
    out, _ = _run_src(hip, src, qo, so, hidden, 256, O.QUANT_INT4, 32)
    _close(out.sum(axis=0, dtype=np.float64), O.qmm(ctx, qo, so, hidden, O.QUANT_INT4, 32)[0], 1e-4, "o projection")


def test_attention_decode_prefetch_workgroups_change_nothing(hip):
    """The prefetching variant (extra workgroups that read other buffers
    into the Infinity Cache) writes the same caches and partials, bit for
    bit, as the plain launch; bad prefetch lists are refused."""
    import ctypes
    lib = hip.open_library()
    heads, kv_heads, d, max_seq, p, slices = 32, 4, 64, 300, 250, 16
    width = (heads + 2 * kv_heads) * d
    qkv = _normal((slices, width), 41)
    ss = np.abs(_normal(5, 42, 50.0)) + 1.0
    cos, sin = L.rope_cache(max_seq, d, 10000.0)
    kc0, vc0 = _normal((kv_heads, max_seq, d), 43), _normal((kv_heads, max_seq, d), 44)
    ch, chs = ctypes.c_int(0), ctypes.c_int(0)
    hip.check(lib.vm_hip_attention_decode_chunks(d, max_seq, ctypes.byref(ch), ctypes.byref(chs)))
    dqkv, dss, dc, dsn = _dev(hip, qkv), _dev(hip, ss), _dev(hip, cos), _dev(hip, sin)
    dpos = _dev(hip, np.array([p], np.int32), np.int32)
    regions = [_dev(hip, _normal(n, 45 + i)) for i, n in enumerate((3 << 18, 12345, 1 << 20))]
    pf = hip.Prefetch()
    for i, r in enumerate(regions):
        pf.ptr[i] = r.addr
        pf.bytes[i] = r.nbytes - (5 if i == 1 else 0)   # a ragged region
    pf.count = len(regions)
    outs = []
    print("case attention_decode_slices prefetch", flush=True)
    for use_pf in (False, True):
        dk, dv = _dev(hip, kc0), _dev(hip, vc0)
        dpart = hip.DeviceBuffer(heads * chs.value * (d + 4) * 4)
        args = (dqkv.ptr, slices, dss.ptr, ss.size, float(2048), 1e-5, dc.ptr, dsn.ptr, dpos.ptr, dk.ptr, dv.ptr,
                dpart.ptr, heads, kv_heads, d, max_seq, 1.0)
        if use_pf:
            hip.check(lib.vm_hip_attention_decode_slices_prefetch_f32(*args, ctypes.byref(pf), None))
        else:
            hip.check(lib.vm_hip_attention_decode_slices_f32(*args, None))
        hip.synchronize()
        n_rec = heads * chs.value * (d + 4)
        outs.append((dk.download(np.float32, kc0.shape), dv.download(np.float32, vc0.shape),
                     dpart.download(np.float32, (n_rec,))))
    (k0, v0, r0), (k1, v1, r1) = outs
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    # records of chunks past the position are never written: compare the written ones
    rec = r0.reshape(heads, chs.value, d + 4)[:, :(p + ch.value) // ch.value]
    assert np.array_equal(rec, r1.reshape(heads, chs.value, d + 4)[:, :(p + ch.value) // ch.value])
    bad = hip.Prefetch()
    bad.count = 5
    dk, dv = _dev(hip, kc0), _dev(hip, vc0)
    dpart = hip.DeviceBuffer(heads * chs.value * (d + 4) * 4)
    args = (dqkv.ptr, slices, dss.ptr, ss.size, float(2048), 1e-5, dc.ptr, dsn.ptr, dpos.ptr, dk.ptr, dv.ptr,
            dpart.ptr, heads, kv_heads, d, max_seq, 1.0)
    assert lib.vm_hip_attention_decode_slices_prefetch_f32(*args, ctypes.byref(bad), None) != 0
    bad.count = 1
    bad.bytes[0] = 64   # non-empty region without a pointer
    assert lib.vm_hip_attention_decode_slices_prefetch_f32(*args, ctypes.byref(bad), None) != 0


def test_swiglu_source_applies_the_norm_scale_and_scaled_slice_sum(hip):
    import ctypes
    k, n, sl_in = 512, 256, 4
    q, s = _pack(k, n, O.QUANT_INT4, 32, 31)
    gu = _normal((sl_in, 2 * k), 8)
    ss = np.array([100.0, 50.0, 25.0], np.float32)
    iv = np.float32(1.0 / np.sqrt(ss.sum(dtype=np.float32) / np.float32(700.0) + np.float32(1e-5)))
    g, u = gu[0, :k].copy(), gu[0, k:].copy()
    for i in range(1, sl_in):
        g, u = (g + gu[i, :k]).astype(np.float32), (u + gu[i, k:]).astype(np.float32)
    x = L.silu_mul((g * iv).astype(np.float32), (u * iv).astype(np.float32))
    dgu, dss = _dev(hip, gu), _dev(hip, ss)
    src = _src(hip, kind=hip.GEMV_SRC_SWIGLU, slices=sl_in, act=dgu.addr, ss_in=dss.addr, ss_count=3, ss_dim=700.0,
               eps=1e-5)
    out, sl = _run_src(hip, src, q, s, k, n, O.QUANT_INT4, 32)
    _close(out.sum(axis=0, dtype=np.float64), O.qmm(x[None], q, s, k, O.QUANT_INT4, 32)[0], TOL, "swiglu")
    # slices_sum_scaled: the projection's slices times the same scale
    do = hip.DeviceBuffer(n * 4)
    dsl = _dev(hip, out)
    hip.check(hip.open_library().vm_hip_slices_sum_scaled_f32(dsl.ptr, sl, n, dss.ptr, 3, 700.0, 1e-5, do.ptr, None))
    tot = out[0].copy()
    for i in range(1, sl):
        tot = (tot + out[i]).astype(np.float32)
    _close(do.download(np.float32, (n,)), tot * iv, 1e-6, "scaled sum")
