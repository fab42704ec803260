"""GPU quantized matmul vs the oracle (the reference CPU backend's
algorithm), through the C ABI.

Contract: max|C_hip - C_ref| <= 1e-3 * max|C_ref| (fp32 accumulation).  The
fp32 GEMV path (rows_m <= 4) and the config-3 GEMMs (activations at 22
significant bits, codes exact, scales applied in fp32) are held to
1e-5 * max|C_ref| as well, which a dropped term, wrong nibble or wrong
scale index would break.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
import ref_inputs

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_GEMV = 1e-5     # fp32 GEMV path


def _normal(shape, seed, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def _check(out, ref, tol):
    ref = np.asarray(ref, np.float64)
    err = np.abs(out.astype(np.float64) - ref).max()
    bound = tol * max(np.abs(ref).max(), 1e-30)
    assert err <= bound, f"max abs err {err:.3e} > {bound:.3e}"


def _int8(k, n, seed):
    return O.quantize_int8(_normal((k, n), seed, 0.02))


def _int4(k, n, seed, block=32):
    return O.quantize_int4(_normal((k, n), seed, 0.02), block)


def test_config1_int8_gemv_smollm2_up_proj(hip):
    # W [1536, 576] (HF [out, in]) -> packed as [K=576, N=1536].
    w = _normal((1536, 576), 1, 0.02).T.copy()
    q, s = O.quantize_int8(w)
    x = _normal((1, 576), 2)
    ref = O.qmm(x, q, s, 576, O.QUANT_INT8, 0)
    out = hip.run_qmm(x, q, s, 576, hip.QUANT_INT8, 0)
    _check(out, ref, TOL_GEMV)


@pytest.mark.parametrize("k,n", [(2048, 2048), (2048, 256), (2048, 5632), (5632, 2048), (2048, 32000)])
def test_config2_int4_gemv_tinyllama_shapes(hip, k, n):
    p, s = _int4(k, n, k + n)
    x = _normal((1, k), n)
    ref = O.qmm(x, p.view(np.int8), s, k, O.QUANT_INT4, 32)
    out = hip.run_qmm(x, p, s, k, hip.QUANT_INT4, 32)
    _check(out, ref, TOL_GEMV)


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("qt", ["int8", "int4"])
def test_small_m_gemv(hip, m, qt):
    k, n = 960, 2560
    x = _normal((m, k), m)
    if qt == "int8":
        q, s = _int8(k, n, 5)
        ref = O.qmm(x, q, s, k, O.QUANT_INT8, 0)
        out = hip.run_qmm(x, q, s, k, hip.QUANT_INT8, 0)
    else:
        q, s = _int4(k, n, 6)
        ref = O.qmm(x, q.view(np.int8), s, k, O.QUANT_INT4, 32)
        out = hip.run_qmm(x, q, s, k, hip.QUANT_INT4, 32)
    _check(out, ref, TOL_GEMV)


@pytest.mark.parametrize("m", [16, 128, 512])
@pytest.mark.parametrize("qt", ["int8", "int4"])
def test_config3_prefill(hip, m, qt):
    k, n = 2048, 5632
    x = _normal((m, k), m + 1)
    if qt == "int8":
        q, s = _int8(k, n, 31)
        w = O.dequantize_int8(q, s)
        out = hip.run_qmm(x, q, s, k, hip.QUANT_INT8, 0)
    else:
        q, s = _int4(k, n, 32)
        w = O.dequantize_int4(q, s, k, 32)
        out = hip.run_qmm(x, q, s, k, hip.QUANT_INT4, 32)
    ref = x.astype(np.float64) @ w.astype(np.float64)
    if m == 16:  # the oracle itself finishes in seconds here
        ref_o = O.qmm(x, q.view(np.int8), s, k, O.QUANT_INT4 if qt == "int4" else O.QUANT_INT8,
                      32 if qt == "int4" else 0)
        _check(ref_o, ref, 1e-5)
    _check(out, ref, TOL)
    _check(out, ref, 1e-5)


@pytest.mark.parametrize("qt", ["int4", "int8"])
def test_output_of_more_than_2gib(hip, qt):
    """A 4100 x 131072 fp32 output (2.05 GiB) on the wide MFMA kernel, which
    addresses C from a 64-bit base per 128-row tile: rows on both sides of
    the 2 GiB mark match the reference loop."""
    m, k, n = 4100, 32, 131072
    x = _normal((m, k), 71)
    if qt == "int4":
        q, s = _int4(k, n, 72)
        hq, oq, blk = hip.QUANT_INT4, O.QUANT_INT4, 32
    else:
        q, s = _int8(k, n, 73)
        hq, oq, blk = hip.QUANT_INT8, O.QUANT_INT8, 0
    da = hip.DeviceBuffer.from_array(x)
    dw = hip.DeviceBuffer.from_array(np.ascontiguousarray(q).view(np.int8))
    ds = hip.DeviceBuffer.from_array(s)
    dc = hip.DeviceBuffer(m * n * 4)
    print(f"case qmm output {m}x{n} ({m * n * 4 / 2**30:.2f} GiB) qt={qt}", flush=True)
    hip.qmm_f32(da.addr, dw.addr, ds.addr, dc.addr, m, k, n, hq, blk)
    hip.synchronize()
    lib = hip.open_library()
    for r0 in (0, 2047, 4094):   # row 4096 starts at 2 GiB
        rows = np.empty((6 if r0 == 4094 else 2, n), np.float32)
        hip.check(lib.vm_hip_memcpy_d2h(rows.ctypes.data, ctypes.c_void_p(dc.addr + r0 * n * 4), rows.nbytes, None))
        ref = O.qmm(x[r0:r0 + rows.shape[0]], q.view(np.int8), s, k, oq, blk)
        _check(rows, ref, 1e-5)


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("k,n", [(64, 64), (128, 256), (576, 576), (576, 1536)])
def test_reference_test_matrix_int8(hip, m, k, n):
    # tests/test_quantization.cpp:140-207 / :310-374 inputs; < 1e-4 absolute.
    w = ref_inputs.generate_random_weights(k, n)
    a = ref_inputs.generate_activations(m, k)
    q, s = O.quantize_int8(w)
    ref = O.qmm(a, q, s, k, O.QUANT_INT8, 0)
    out = hip.run_qmm(a, q, s, k, hip.QUANT_INT8, 0)
    assert np.abs(out - ref).max() < 1e-4 if m <= 4 else np.abs(out - ref).max() < 1e-3 * np.abs(ref).max()


@pytest.mark.parametrize("m,k,n,qt,block", [
    (1, 31, 64, "int4", 32),      # K tail, odd K
    (2, 33, 48, "int4", 32),
    (1, 100, 1024, "int4", 64),   # block 64
    (1, 256, 4096, "int4", 128),
    (3, 70, 20, "int8", 0),       # N % 16 != 0, N % 4 == 0
    (1, 70, 13, "int8", 0),       # odd N -> generic kernel
    (1, 64, 13, "int4", 32),
    (2, 96, 512, "int8", 32),     # INT8 blockwise
    (1, 96, 512, "int8", 16),     # block not multiple of 32 -> generic
    (1, 64, 40, "int4", 8),
    (5, 64, 40, "int4", 0),       # INT4 block 0 means 32
    (1, 96, 1024, "int4", 0),
    (1, 1, 1, "int8", 0),
])
def test_edge_shapes(hip, m, k, n, qt, block):
    x = _normal((m, k), k * n)
    w = _normal((k, n), k + n, 0.02)
    if qt == "int8":
        if block:
            nb = (k + block - 1) // block
            q = np.random.default_rng(3).integers(-127, 128, (k, n), dtype=np.int8)
            s = np.random.default_rng(4).random((nb, n)).astype(np.float32)
        else:
            q, s = O.quantize_int8(w)
        ref = O.qmm(x, q, s, k, O.QUANT_INT8, block)
        out = hip.run_qmm(x, q, s, k, hip.QUANT_INT8, block)
    else:
        q, s = O.quantize_int4(w, block or 32)
        ref = O.qmm(x, q.view(np.int8), s, k, O.QUANT_INT4, block)
        out = hip.run_qmm(x, q, s, k, hip.QUANT_INT4, block)
    _check(out, ref, TOL_GEMV if m <= 4 else TOL)


def test_k_zero_writes_zeros_and_empty_is_noop(hip):
    dc = hip.DeviceBuffer.from_array(np.full((2, 8), 7.0, np.float32))
    hip.qmm_f32(0, 0, 0, dc.addr, 2, 0, 8, hip.QUANT_INT8, 0)
    assert not dc.download(np.float32, (2, 8)).any()
    hip.qmm_f32(0, 0, 0, 0, 0, 4, 8, hip.QUANT_INT8, 0)   # m == 0
    hip.qmm_f32(0, 0, 0, 0, 2, 4, 0, hip.QUANT_INT8, 0)   # n == 0


def test_invalid_arguments_raise(hip):
    buf = hip.DeviceBuffer(4096)
    with pytest.raises(hip.VmHipError) as e:
        hip.qmm_f32(buf.addr, buf.addr, buf.addr, buf.addr, 1, 8, 8, hip.QUANT_INT4, 3)
    assert e.value.status == hip.EINVAL and "even" in str(e.value)
    with pytest.raises(hip.VmHipError):
        hip.qmm_f32(buf.addr, buf.addr, buf.addr, buf.addr, 1, 8, 8, 7, 0)
    with pytest.raises(hip.VmHipError):
        hip.qmm_f32(0, buf.addr, buf.addr, buf.addr, 1, 8, 8, hip.QUANT_INT8, 0)


def test_deterministic_and_stream_workspace_reuse(hip):
    k, n = 2048, 2048
    p, s = _int4(k, n, 77)
    x = _normal((1, k), 78)
    da, dp, ds = (hip.DeviceBuffer.from_array(v) for v in (x, p, s))
    outs = []
    streams = [hip.Stream(), hip.Stream()]
    dcs = [hip.DeviceBuffer(n * 4) for _ in range(4)]
    # interleave calls on two streams and a smaller shape in between
    p2, s2 = _int4(4096, 256, 79)
    x2 = _normal((1, 4096), 80)
    da2, dp2, ds2 = (hip.DeviceBuffer.from_array(v) for v in (x2, p2, s2))
    dsmall = hip.DeviceBuffer(256 * 4)
    for i, dc in enumerate(dcs):
        st = streams[i % 2]
        hip.qmm_f32(da.addr, dp.addr, ds.addr, dc.addr, 1, k, n, hip.QUANT_INT4, 32, st)
        hip.qmm_f32(da2.addr, dp2.addr, ds2.addr, dsmall.addr, 1, 4096, 256, hip.QUANT_INT4, 32, st)
    for st in streams:
        st.synchronize()
    outs = [dc.download(np.float32, (n,)) for dc in dcs]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    ref = O.qmm(x, p.view(np.int8), s, k, O.QUANT_INT4, 32)[0]
    _check(outs[0], ref, TOL_GEMV)
    ref2 = O.qmm(x2, p2.view(np.int8), s2, 4096, O.QUANT_INT4, 32)[0]
    _check(dsmall.download(np.float32, (256,)), ref2, TOL_GEMV)


@pytest.mark.parametrize("k,n", [(2048, 5632), (5632, 2048), (2560, 960)])
def test_split_tree_zero_columns(hip, k, n):
    """Split-K shapes (the pair-word tree) with all-zero weight columns, so
    every split's sum for them is zero (its fp32 bits are 0, the pattern
    an empty pair-word half holds before encoding): the tree must still see
    every split arrive, those outputs are exactly zero, and repeated calls
    are bit-identical."""
    w = _normal((k, n), 91, 0.02)
    w[:, ::7] = 0.0
    x = -np.abs(_normal((1, k), 92))
    for qt in ("int8", "int4"):
        if qt == "int8":
            q, s = O.quantize_int8(w)
            ref = O.qmm(x, q, s, k, O.QUANT_INT8, 0)
            out = hip.run_qmm(x, q, s, k, hip.QUANT_INT8, 0)
        else:
            q, s = O.quantize_int4(w, 32)
            ref = O.qmm(x, q.view(np.int8), s, k, O.QUANT_INT4, 32)
            out = hip.run_qmm(x, q, s, k, hip.QUANT_INT4, 32)
        assert not out[0, ::7].any(), qt
        _check(out, ref, TOL_GEMV)
        again = hip.run_qmm(x, q, s, k, hip.QUANT_INT8 if qt == "int8" else hip.QUANT_INT4, 0 if qt == "int8" else 32)
        assert np.array_equal(out.view(np.uint32), again.view(np.uint32)), qt


def test_graph_keeps_workspace_after_growth(hip):
    """A split-K GEMV captured in a graph still replays correctly after an
    eager call on the same stream has grown the stream's workspace (the
    graph holds the old buffer's address, which must stay allocated)."""
    k, n = 2048, 2048
    p, s = _int4(k, n, 81)
    x = _normal((1, k), 82)
    da, dp, ds = (hip.DeviceBuffer.from_array(v) for v in (x, p, s))
    st = hip.Stream()
    d_eager, d_graph = hip.DeviceBuffer(n * 4), hip.DeviceBuffer(n * 4)
    hip.qmm_f32(da.addr, dp.addr, ds.addr, d_eager.addr, 1, k, n, hip.QUANT_INT4, 32, st)   # sizes the workspace
    g = hip.Graph(st)
    g.begin()
    hip.qmm_f32(da.addr, dp.addr, ds.addr, d_graph.addr, 1, k, n, hip.QUANT_INT4, 32, st)
    g.end()
    # The two-pass INT8 pack of a 2048 x 8192 matrix keeps 64 x 8192 row
    # partials in the same workspace: more than the GEMV sized it for.
    rows, cols = 2048, 8192
    w = _normal((rows, cols), 83, 0.02)
    dw = hip.DeviceBuffer.from_array(w)
    dq, dsc = hip.DeviceBuffer(rows * cols), hip.DeviceBuffer(cols * 4)
    hip.pack_int8(dw.addr, dq.addr, dsc.addr, rows, cols, st)
    st.synchronize()
    filler = hip.DeviceBuffer.from_array(np.full(1 << 22, 0xFF, np.uint8))   # reuses freed memory, if any
    eager = d_eager.download(np.float32, (n,))
    for _ in range(3):
        d_graph.upload(np.zeros(n, np.float32))
        g.launch()
        st.synchronize()
        assert np.array_equal(d_graph.download(np.float32, (n,)).view(np.uint32), eager.view(np.uint32))
    g.close()
    st.close()
    del filler
    q_ref, s_ref = O.quantize_int8(w)
    assert np.array_equal(dq.download(np.int8, (rows, cols)), q_ref.view(np.int8))
    assert np.array_equal(dsc.download(np.float32, (cols,)).view(np.uint32), s_ref.view(np.uint32))
    _check(eager, O.qmm(x, p.view(np.int8), s, k, O.QUANT_INT4, 32)[0], TOL_GEMV)


@pytest.mark.parametrize("a_dt,s_dt", [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
def test_mixed_dtype_keys(hip, a_dt, s_dt):
    # quantized_matmul.cpp:363-367 dtype keys; outputs rounded like dtype.h.
    m, k, n = 2, 128, 96
    rng = np.random.default_rng(12)
    q, s = O.quantize_int8((rng.standard_normal((k, n)) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    codes = {"f16": O.F16, "bf16": O.BF16, "f32": O.F32}
    a_bits = O.f32_to_f16_bits(a) if a_dt == "f16" else O.f32_to_bf16_bits(a)
    s_arr = s if s_dt == "f32" else (O.f32_to_f16_bits(s) if s_dt == "f16" else O.f32_to_bf16_bits(s))
    ref = O.qmm_mixed(a_bits, codes[a_dt], q, s_arr, codes[s_dt], codes[a_dt], k, O.QUANT_INT8, 0)
    da = hip.DeviceBuffer.from_array(a_bits)
    dq = hip.DeviceBuffer.from_array(q)
    ds = hip.DeviceBuffer.from_array(s_arr)
    dc = hip.DeviceBuffer(m * n * 2)
    dtc = {"f16": hip.DTYPE_F16, "bf16": hip.DTYPE_BF16, "f32": hip.DTYPE_F32}
    hip.qmm(da.addr, dtc[a_dt], dq.addr, ds.addr, dtc[s_dt], dc.addr, dtc[a_dt], m, k, n, hip.QUANT_INT8, 0)
    out = dc.download(np.uint16, (m, n))
    to32 = (lambda b: b.view(np.float16).astype(np.float32)) if a_dt == "f16" else \
        (lambda b: (b.astype(np.uint32) << 16).view(np.float32))
    # one half-precision ulp of the output
    ulp = 2.0 ** -10 if a_dt == "f16" else 2.0 ** -7
    assert np.abs(to32(out) - to32(ref)).max() <= ulp * np.abs(to32(ref)).max()


def test_injected_failure_is_reported(hip, monkeypatch):
    monkeypatch.setenv("VELOMIND_FAIL_BACKEND", "HIP:QuantizedMatMul:launch")
    buf = hip.DeviceBuffer(4096)
    with pytest.raises(hip.VmHipError) as e:
        hip.qmm_f32(buf.addr, buf.addr, buf.addr, buf.addr, 1, 8, 8, hip.QUANT_INT8, 0)
    assert e.value.status == hip.EINJECTED and "injected failure" in str(e.value)
