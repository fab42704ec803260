"""The graph compiler's fused chains on DeviceType::HIP (graph_compiler.cpp
fuse_steps, kernel.h FusedKind).

Each fused kernel is compared with the chain of single-operator launches it
replaces, bit for bit, through the C ABI: the decode attention chain
(RepeatKV, Transpose, MatMul, Softmax, MatMul), QuantizedMatMul followed by
its residual Add, RMSNorm feeding sibling QuantizedMatMuls, RoPE with the
KV-cache appends, and the SwiGLU Mul(Mul(Sigmoid(g), g), u).  Then the graph
engine (the reference engine's loop, a Graph per call) decodes with fusion
on (the default) and with VELOMIND_GRAPH_FUSE=0, and the logits must be
identical, for both attention forms of the reference layer and every
quantization.  The unfused chain itself is held against the oracle by
tests/test_hip_llama_e2e.py and tests/test_hip_llama_full.py.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int, c_int64

import numpy as np
import pytest

import llama_oracle as L

pytestmark = pytest.mark.gpu


def _dev(H, a):
    return H.DeviceBuffer.from_array(np.ascontiguousarray(a))


# V copied into LDS (s * d fits: s = 1 ... 400, partial last 1 KiB blocks
# included) and V read from global memory (s = 775 and 1000 overflow LDS;
# d = 18 is not a multiple of 4).
@pytest.mark.parametrize("hq,hkv,s,d", [(8, 2, 37, 64), (15, 5, 129, 64), (15, 5, 256, 64), (15, 5, 400, 64),
                                         (32, 4, 775, 64), (4, 4, 1, 16), (6, 3, 17, 20), (4, 2, 33, 18),
                                         (2, 1, 1000, 128)])
def test_attention_decode_chain_matches_the_unfused_chain(hip, hq, hkv, s, d):
    H = hip
    lib = H.open_library()
    print(f"case attention chain hq={hq} hkv={hkv} s={s} d={d}", flush=True)
    rng = np.random.default_rng(hq * 1000 + s)
    q = rng.standard_normal((hq, 1, d), dtype=np.float32)
    k = rng.standard_normal((hkv, s, d), dtype=np.float32)
    v = rng.standard_normal((hkv, s, d), dtype=np.float32)
    dq, dk, dv = _dev(H, q), _dev(H, k), _dev(H, v)
    rep = hq // hkv
    kr, vr = H.DeviceBuffer(hq * s * d * 4), H.DeviceBuffer(hq * s * d * 4)
    kt, sc, p = H.DeviceBuffer(hq * s * d * 4), H.DeviceBuffer(hq * s * 4), H.DeviceBuffer(hq * s * 4)
    ref, out = H.DeviceBuffer(hq * d * 4), H.DeviceBuffer(hq * d * 4)
    H.check(lib.vm_hip_repeat_kv_f32(dk.ptr, kr.ptr, 1, hkv, rep, s * d, None))
    H.check(lib.vm_hip_repeat_kv_f32(dv.ptr, vr.ptr, 1, hkv, rep, s * d, None))
    shape = (c_int64 * 3)(hq, s, d)
    perm = (c_int * 3)(0, 2, 1)
    H.check(lib.vm_hip_transpose_f32(kr.ptr, kt.ptr, 3, ctypes.cast(shape, ctypes.c_void_p),
                                     ctypes.cast(perm, ctypes.c_void_p), None))
    H.check(lib.vm_hip_matmul_f32(dq.ptr, kt.ptr, sc.ptr, hq, 1, d, s, None))
    H.check(lib.vm_hip_softmax_f32(sc.ptr, p.ptr, hq, s, 1, None))
    H.check(lib.vm_hip_matmul_f32(p.ptr, vr.ptr, ref.ptr, hq, 1, s, d, None))
    H.check(lib.vm_hip_attention_decode_chain_f32(dq.ptr, dk.ptr, dv.ptr, out.ptr, hq, hkv, s, d, d, None))
    H.synchronize()
    a = out.download(np.float32, (hq, d))
    b = ref.download(np.float32, (hq, d))
    assert np.all(np.isfinite(b))
    assert a.tobytes() == b.tobytes(), f"max diff {np.abs(a - b).max():.3e}"


def test_attention_decode_chain_rejects_bad_shapes(hip):
    lib = hip.open_library()
    buf = hip.DeviceBuffer(4096)
    for hq, hkv, s, d in [(6, 4, 8, 16), (4, 0, 8, 16), (4, 4, 0, 16), (4, 4, 16380, 16)]:
        assert lib.vm_hip_attention_decode_chain_f32(buf.ptr, buf.ptr, buf.ptr, buf.ptr, hq, hkv, s, d, d, None) != 0


@pytest.mark.parametrize("m,k,n,qt,blk", [
    (1, 960, 960, 1, 0), (1, 2560, 960, 1, 0), (1, 2048, 2048, 2, 32), (1, 5632, 2048, 2, 32),
    (2, 2048, 256, 2, 32), (3, 576, 1536, 1, 0), (4, 2048, 2048, 1, 32), (8, 2048, 256, 2, 32),
    (1, 64, 40, 2, 32)])
def test_qmm_add_matches_qmm_then_add(hip, m, k, n, qt, blk):
    H = hip
    lib = H.open_library()
    print(f"case qmm+add m={m} k={k} n={n} qt={qt} blk={blk}", flush=True)
    rng = np.random.default_rng(m * 7919 + k + n)
    rows = (k + 1) // 2 if qt == 2 else k
    codes = rng.integers(-128, 128, size=(rows, n), dtype=np.int8)
    nb = (k + blk - 1) // blk if blk > 0 else 1
    scales = (rng.random((nb, n), dtype=np.float32) * 0.02).astype(np.float32)
    a = rng.standard_normal((m, k), dtype=np.float32)
    h = rng.standard_normal((m, n), dtype=np.float32)
    da, dw, ds, dh = _dev(H, a), _dev(H, codes), _dev(H, scales), _dev(H, h)
    ref, out = H.DeviceBuffer(m * n * 4), H.DeviceBuffer(m * n * 4)
    for _ in range(2):   # a second call reuses the split-K words the first cleared
        H.check(lib.vm_hip_qmm_f32(da.ptr, dw.ptr, ds.ptr, ref.ptr, m, k, n, qt, blk, None))
        H.check(lib.vm_hip_elementwise_f32(H.EW_ADD, dh.ptr, ref.ptr, ref.ptr, m * n, None))
        H.check(lib.vm_hip_qmm_add_f32(da.ptr, dw.ptr, ds.ptr, dh.ptr, out.ptr, m, k, n, qt, blk, None))
        H.synchronize()
        x = out.download(np.float32, (m, n))
        y = ref.download(np.float32, (m, n))
        assert x.tobytes() == y.tobytes(), f"max diff {np.abs(x - y).max():.3e}"


@pytest.mark.parametrize("m,k,ns,qt,blk", [
    (1, 960, (960, 320, 320), 1, 0), (1, 2048, (2048, 256, 256), 2, 32), (2, 2048, (5632, 5632), 2, 32),
    (3, 576, (1536,), 1, 0), (4, 960, (2560, 2560), 1, 32), (1, 5632, (2048,), 2, 32),
    (8, 960, (960, 320), 1, 0), (1, 64, (40, 48), 2, 32)])
def test_norm_group_matches_rmsnorm_then_group(hip, m, k, ns, qt, blk):
    H = hip
    lib = H.open_library()
    print(f"case norm group m={m} k={k} ns={ns} qt={qt} blk={blk}", flush=True)
    rng = np.random.default_rng(m * 131 + k + len(ns))
    rows = (k + 1) // 2 if qt == 2 else k
    nb = (k + blk - 1) // blk if blk > 0 else 1
    a = (rng.standard_normal((m, k), dtype=np.float32) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k, dtype=np.float32)).astype(np.float32)
    da, dnw = _dev(H, a), _dev(H, nw)
    hn = H.DeviceBuffer(m * k * 4)
    keep, ref_m, out_m = [], (H.QmmMember * len(ns))(), (H.QmmMember * len(ns))()
    for g, n in enumerate(ns):
        codes = _dev(H, rng.integers(-128, 128, size=(rows, n), dtype=np.int8))
        scales = _dev(H, (rng.random((nb, n), dtype=np.float32) * 0.02).astype(np.float32))
        ref, out = H.DeviceBuffer(m * n * 4), H.DeviceBuffer(m * n * 4)
        keep += [codes, scales, ref, out]
        ref_m[g] = H.QmmMember(codes.addr, scales.addr, ref.addr, n)
        out_m[g] = H.QmmMember(codes.addr, scales.addr, out.addr, n)
    eps = 1e-5
    for _ in range(2):
        H.check(lib.vm_hip_rmsnorm_f32(da.ptr, dnw.ptr, hn.ptr, m, k, ctypes.c_float(eps), None))
        H.check(lib.vm_hip_qmm_group_f32(hn.ptr, m, k, ref_m, len(ns), qt, blk, None))
        H.check(lib.vm_hip_qmm_norm_group_f32(da.ptr, dnw.ptr, ctypes.c_float(eps), m, k, out_m, len(ns), qt, blk,
                                              None))
        H.synchronize()
        for g, n in enumerate(ns):
            x = keep[4 * g + 3].download(np.float32, (m, n))
            y = keep[4 * g + 2].download(np.float32, (m, n))
            assert np.all(np.isfinite(y))
            assert x.tobytes() == y.tobytes(), f"member {g}: max diff {np.abs(x - y).max():.3e}"


@pytest.mark.parametrize("hq,hkv,s,d", [(15, 5, 128, 64), (32, 4, 767, 64), (4, 4, 1, 16), (6, 2, 9, 8)])
def test_rope_append_matches_rope_and_concat(hip, hq, hkv, s, d):
    H = hip
    lib = H.open_library()
    print(f"case rope append hq={hq} hkv={hkv} s={s} d={d}", flush=True)
    rng = np.random.default_rng(s + d)
    arrs = [rng.standard_normal(sh, dtype=np.float32) for sh in
            ((hq, 1, d), (hkv, 1, d), (hkv, 1, d), (hkv, s, d), (hkv, s, d), (1, d // 2), (1, d // 2))]
    q, k, v, pk, pv, cs, sn = (_dev(H, x) for x in arrs)
    qr, kr = H.DeviceBuffer(hq * d * 4), H.DeviceBuffer(hkv * d * 4)
    kc, vc = H.DeviceBuffer(hkv * (s + 1) * d * 4), H.DeviceBuffer(hkv * (s + 1) * d * 4)
    fq, fk, fv = H.DeviceBuffer(hq * d * 4), H.DeviceBuffer(hkv * (s + 1) * d * 4), H.DeviceBuffer(hkv * (s + 1) * d * 4)
    H.check(lib.vm_hip_rope_f32(q.ptr, cs.ptr, sn.ptr, qr.ptr, hq, d, 1, None))
    H.check(lib.vm_hip_rope_f32(k.ptr, cs.ptr, sn.ptr, kr.ptr, hkv, d, 1, None))
    H.check(lib.vm_hip_concat_f32(pk.ptr, kr.ptr, kc.ptr, hkv, s * d, d, None))
    H.check(lib.vm_hip_concat_f32(pv.ptr, v.ptr, vc.ptr, hkv, s * d, d, None))
    H.check(lib.vm_hip_rope_append_f32(q.ptr, k.ptr, v.ptr, pk.ptr, pv.ptr, cs.ptr, sn.ptr, fq.ptr, fk.ptr, fv.ptr,
                                       hq, hkv, s, d, d, None))
    H.synchronize()
    for got, ref, size in ((fq, qr, hq * d), (fk, kc, hkv * (s + 1) * d), (fv, vc, hkv * (s + 1) * d)):
        assert got.download(np.float32, (size,)).tobytes() == ref.download(np.float32, (size,)).tobytes()


@pytest.mark.parametrize("m,k,n,qt,blk,with_add", [
    (1, 2560, 960, 1, 0, True), (1, 5632, 2048, 2, 32, True), (2, 5632, 2048, 2, 32, False),
    (4, 2560, 960, 1, 32, True), (8, 2560, 960, 1, 0, True), (1, 64, 40, 2, 32, True)])
def test_qmm_swiglu_add_matches_the_separate_launches(hip, m, k, n, qt, blk, with_add):
    H = hip
    lib = H.open_library()
    print(f"case swiglu qmm m={m} k={k} n={n} qt={qt} blk={blk} add={with_add}", flush=True)
    rng = np.random.default_rng(m * 17 + k + n)
    rows = (k + 1) // 2 if qt == 2 else k
    nb = (k + blk - 1) // blk if blk > 0 else 1
    g = (rng.standard_normal((m, k), dtype=np.float32) * 3).astype(np.float32)
    u = rng.standard_normal((m, k), dtype=np.float32)
    h = rng.standard_normal((m, n), dtype=np.float32)
    dg, du, dh = _dev(H, g), _dev(H, u), _dev(H, h)
    dw = _dev(H, rng.integers(-128, 128, size=(rows, n), dtype=np.int8))
    ds = _dev(H, (rng.random((nb, n), dtype=np.float32) * 0.02).astype(np.float32))
    act, ref, out = H.DeviceBuffer(m * k * 4), H.DeviceBuffer(m * n * 4), H.DeviceBuffer(m * n * 4)
    for _ in range(2):
        H.check(lib.vm_hip_elementwise_f32(H.EW_SILU_MUL, dg.ptr, du.ptr, act.ptr, m * k, None))
        H.check(lib.vm_hip_qmm_f32(act.ptr, dw.ptr, ds.ptr, ref.ptr, m, k, n, qt, blk, None))
        if with_add:
            H.check(lib.vm_hip_elementwise_f32(H.EW_ADD, dh.ptr, ref.ptr, ref.ptr, m * n, None))
        H.check(lib.vm_hip_qmm_swiglu_add_f32(dg.ptr, du.ptr, dw.ptr, ds.ptr, dh.ptr if with_add else None,
                                              out.ptr, m, k, n, qt, blk, None))
        H.synchronize()
        x = out.download(np.float32, (m, n))
        y = ref.download(np.float32, (m, n))
        assert np.all(np.isfinite(y))
        assert x.tobytes() == y.tobytes(), f"max diff {np.abs(x - y).max():.3e}"


def test_silu_mul_matches_sigmoid_mul_mul(hip):
    H = hip
    lib = H.open_library()
    n = 3 * 2560 + 7
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(n, dtype=np.float32) * 4).astype(np.float32)
    u = rng.standard_normal(n, dtype=np.float32)
    g[:4] = [0.0, -0.0, 88.0, -104.0]
    dg, du = _dev(H, g), _dev(H, u)
    t1, t2, ref, out = (H.DeviceBuffer(n * 4) for _ in range(4))
    H.check(lib.vm_hip_elementwise_f32(H.EW_SIGMOID, dg.ptr, None, t1.ptr, n, None))
    H.check(lib.vm_hip_elementwise_f32(H.EW_MUL, t1.ptr, dg.ptr, t2.ptr, n, None))
    H.check(lib.vm_hip_elementwise_f32(H.EW_MUL, t2.ptr, du.ptr, ref.ptr, n, None))
    H.check(lib.vm_hip_elementwise_f32(H.EW_SILU_MUL, dg.ptr, du.ptr, out.ptr, n, None))
    H.synchronize()
    assert out.download(np.float32, (n,)).tobytes() == ref.download(np.float32, (n,)).tobytes()


def _gqa_model(seed=19):
    # head_dim 64, 3 query heads per KV head (SmolLM2's grouping)
    cfg = L.LlamaConfig(vocab_size=300, hidden_size=384, intermediate_size=640, num_layers=3, num_heads=6,
                        num_kv_heads=2, rms_norm_eps=1e-5, rope_theta=100000.0)
    rng = np.random.default_rng(seed)
    n = lambda *s: (rng.standard_normal(s) * 0.05).astype(np.float32)  # noqa: E731
    lin = lambda k, m: L._lin(n(k, m))                                   # noqa: E731
    h, kv, i = cfg.hidden_size, cfg.kv_heads * cfg.head_dim, cfg.intermediate_size
    w = L.LlamaWeights(embed=n(cfg.vocab_size, h) * 10, final_norm=1 + n(h), lm_head=lin(h, cfg.vocab_size))
    for _ in range(cfg.num_layers):
        w.attn_norm.append(1 + n(h))
        w.ffn_norm.append(1 + n(h))
        w.wq.append(lin(h, h))
        w.wk.append(lin(h, kv))
        w.wv.append(lin(h, kv))
        w.wo.append(lin(h, h))
        w.gate.append(lin(h, i))
        w.up.append(lin(h, i))
        w.down.append(lin(i, h))
    return cfg, w


@pytest.mark.parametrize("fused_attention", [False, True])
@pytest.mark.parametrize("qt,block", [(0, 0), (1, 0), (2, 32)])
def test_graph_engine_fusion_changes_no_logit(hip, monkeypatch, qt, block, fused_attention):
    from velomind_hip import llama as VL

    cfg, w = _gqa_model()
    dev = VL.Weights.from_oracle(cfg, w)
    print(f"case graph fusion qt={qt} fused_attention={fused_attention}", flush=True)
    prompt = [7, 3, 250]
    steps = ((3, 11), (4, 12), (5, 13), (6, 200))

    def run():
        s = VL.Session(dev, VL.ENGINE_GRAPH, qt, block, fused_attention)
        out = [s.prefill(prompt)]
        for pos, tok in steps:
            out.append(s.forward_step(tok, pos))
        s.close()
        return out

    fused = run()
    monkeypatch.setenv("VELOMIND_GRAPH_FUSE", "0")
    plain = run()
    monkeypatch.delenv("VELOMIND_GRAPH_FUSE")
    for i, (a, b) in enumerate(zip(fused, plain)):
        a = np.asarray(a, np.float32)
        b = np.asarray(b, np.float32)
        assert np.all(np.isfinite(b)) and np.abs(b).max() > 0
        assert a.tobytes() == b.tobytes(), f"call {i}: max diff {np.abs(a - b).max():.3e}"
