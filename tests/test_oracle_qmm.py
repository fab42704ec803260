"""Pins the oracle's CPU QuantizedMatMul restatement
(src/cpu/ops/quantized_matmul.cpp) and the half-precision converters
(include/velomind/dtype.h).

INT8 per-channel is pinned by the reference's own tests on their exact
inputs (tests/test_quantization.cpp:140-241).  No reference test executes
INT4 or blockwise INT8, so those are pinned by closed forms: codes decoded
independently in numpy, per-(block, column) scales that differ by powers of
two (a transposed scale index or a wrong block boundary changes the
result), odd K and the nibble select by row parity.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import ref_inputs


def _unpack_int4(packed: np.ndarray, rows: int) -> np.ndarray:
    nib = np.stack([packed & 0xF, packed >> 4], axis=1).reshape(-1, packed.shape[1])[:rows]
    return np.where(nib >= 8, nib.astype(np.int64) - 16, nib.astype(np.int64))


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("k,n", [(64, 64), (128, 256), (576, 576), (576, 1536)])
def test_reference_int8_qmm_vs_dequant_matmul(m, k, n):
    # tests/test_quantization.cpp:140-207: |QMM - MatMul(A, dequant(W))| < 1e-4.
    w = ref_inputs.generate_random_weights(k, n)
    a = ref_inputs.generate_activations(m, k)
    q, s = O.quantize_int8(w)
    ref = a.astype(np.float64) @ O.dequantize_int8(q, s).astype(np.float64)
    out = O.qmm(a, q, s, k, O.QUANT_INT8, 0)
    assert np.abs(out - ref).max() < 1e-4


@pytest.mark.parametrize("quant,block", [(O.QUANT_INT8, 0), (O.QUANT_INT8, 32), (O.QUANT_INT8, 7),
                                         (O.QUANT_INT4, 32), (O.QUANT_INT4, 0), (O.QUANT_INT4, 2), (O.QUANT_INT4, 64)])
@pytest.mark.parametrize("m,k,n", [(2, 64, 16), (3, 101, 37), (5, 576, 1536), (2, 2048, 96), (4, 0, 8), (3, 33, 1)])
def test_row_major_loop_is_the_scalar_reference_bit_for_bit(quant, block, m, k, n):
    """vmo_qmm_2d_f32 runs the scalar reference's per-element arithmetic in
    row-major order (the loop the full-size exact oracle needs); every
    element must come out bit-identical to the reference's column loop,
    including odd K, tails of blocks, per-channel INT8 and values of every
    magnitude (an fp32 reassociation or a contraction would show)."""
    rng = np.random.default_rng(m * 1000 + k + n + block)
    if quant == O.QUANT_INT4:
        q = rng.integers(0, 256, ((k + 1) // 2, n), dtype=np.uint8).view(np.int8)
        nb = -(-k // (block if block > 0 else 32))
    else:
        q = rng.integers(-128, 128, (k, n), dtype=np.int8)
        nb = -(-k // block) if block > 0 else 1
    s = (np.exp2(rng.integers(-20, 20, (max(nb, 1), n))) * rng.uniform(0.5, 1.0, (max(nb, 1), n))).astype(np.float32)
    a = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-30, 30, (m, k)))).astype(np.float32)
    fast = O.qmm(a, q, s, k, quant, block)
    ref = O.qmm_scalar(a, q, s, k, quant, block)
    assert np.array_equal(fast.view(np.uint32), ref.view(np.uint32))


def test_reference_avx2_decode_vs_scalar():
    # tests/test_quantization.cpp:209-241
    k, n = 576, 1536
    q, s = O.quantize_int8(ref_inputs.generate_random_weights(k, n))
    a = ref_inputs.generate_activations(1, k)
    stream = O.qmm_decode_int8(a, q, s)
    scalar = O.qmm_scalar(a, q, s, k, O.QUANT_INT8, 0)[0]
    assert np.abs(stream - scalar).max() < 1e-4


def test_decode_path_only_for_per_channel_int8():
    # quantized_matmul.cpp:203-208: INT4, blockwise INT8 and strided A decline.
    q = np.zeros((4, 4), np.int8)
    a = np.zeros(4, np.float32)
    L, p = O.lib(), (lambda x: x.ctypes.data)
    assert L.vmo_qmm_decode_int8(p(a), p(q), p(a), p(a), 4, 4, 1, 4, 1, O.QUANT_INT4, 32) == 0
    assert L.vmo_qmm_decode_int8(p(a), p(q), p(a), p(a), 4, 4, 1, 4, 1, O.QUANT_INT8, 32) == 0
    assert L.vmo_qmm_decode_int8(p(a), p(q), p(a), p(a), 2, 4, 2, 4, 1, O.QUANT_INT8, 0) == 0
    assert L.vmo_qmm_decode_int8(p(a), p(q), p(a), p(a), 4, 4, 1, 4, 1, O.QUANT_INT8, 0) == 1


@pytest.mark.parametrize("m,k,n,block", [(1, 64, 8, 32), (3, 100, 5, 32), (2, 7, 3, 2), (1, 2048, 16, 32),
                                         (5, 96, 11, 64), (1, 31, 4, 32)])
def test_int4_closed_form(m, k, n, block):
    rng = np.random.default_rng(k * 31 + n)
    packed = rng.integers(0, 256, size=((k + 1) // 2, n), dtype=np.uint8)
    if k % 2:
        packed[-1] &= 0x0F
    nb = (k + block - 1) // block
    # power-of-two scales that differ per (block, column)
    scales = np.ldexp(np.ones((nb, n), np.float32), (np.arange(nb)[:, None] % 5 - 2) + (np.arange(n)[None, :] % 3)).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    codes = _unpack_int4(packed, k).astype(np.float64)
    w = codes * np.repeat(scales.astype(np.float64), block, axis=0)[:k]
    ref = a.astype(np.float64) @ w
    out = O.qmm(a, packed.view(np.int8), scales, k, O.QUANT_INT4, block)
    assert np.abs(out - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    # the same data with the scale table transposed in memory must disagree
    if nb > 1 and n > 1 and nb != n:
        bad = O.qmm(a, packed.view(np.int8), np.ascontiguousarray(scales.T).reshape(nb, n), k, O.QUANT_INT4, block)
        assert np.abs(bad - ref).max() > 1e-3 * np.abs(ref).max()


def test_int4_nibble_parity_known_answer():
    # one byte 0x9F: low nibble -1 (row 0), high nibble -7 (row 1); scale 0.5
    packed = np.array([[0x9F]], np.uint8)
    a = np.array([[2.0, 3.0]], np.float32)
    out = O.qmm(a, packed.view(np.int8), np.array([[0.5]], np.float32), 2, O.QUANT_INT4, 32)
    assert out[0, 0] == np.float32((2.0 * -1 + 3.0 * -7) * 0.5)


def test_int4_block_size_zero_defaults_to_32():
    # quantized_matmul.cpp:67: block_size <= 0 means 32-row blocks for INT4.
    rng = np.random.default_rng(5)
    k, n = 96, 6
    packed = rng.integers(0, 256, size=(k // 2, n), dtype=np.uint8).view(np.int8)
    s = rng.random((3, n)).astype(np.float32)
    a = rng.standard_normal((2, k)).astype(np.float32)
    assert np.array_equal(O.qmm(a, packed, s, k, O.QUANT_INT4, 0), O.qmm(a, packed, s, k, O.QUANT_INT4, 32))


@pytest.mark.parametrize("m,k,n,block", [(2, 64, 8, 32), (1, 70, 5, 16), (4, 33, 3, 8)])
def test_int8_blockwise_closed_form(m, k, n, block):
    rng = np.random.default_rng(m + k + n)
    q = rng.integers(-127, 128, size=(k, n), dtype=np.int8)
    nb = (k + block - 1) // block
    s = np.ldexp(np.ones((nb, n), np.float32), np.arange(nb * n).reshape(nb, n) % 7 - 3).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    ref = a.astype(np.float64) @ (q.astype(np.float64) * np.repeat(s.astype(np.float64), block, axis=0)[:k])
    out = O.qmm(a, q, s, k, O.QUANT_INT8, block)
    assert np.abs(out - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_int8_per_channel_closed_form_m_gt_1():
    rng = np.random.default_rng(11)
    m, k, n = 7, 45, 13
    q = rng.integers(-127, 128, size=(k, n), dtype=np.int8)
    s = rng.random(n).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    ref = (a.astype(np.float64) @ q.astype(np.float64)) * s.astype(np.float64)
    assert np.abs(O.qmm(a, q, s, k, O.QUANT_INT8, 0) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    L = O.lib()
    ours = np.array([L.vmo_f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(ours[np.isnan(ref)]).all() and np.array_equal(ours[np.isinf(ref)], ref[np.isinf(ref)])


def test_f32_to_f16_matches_ieee_rne_in_normal_range():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 100,
                        np.float32([65504, 65519.99, 65520, 1e6, -1e6, 6.1035156e-05, 0.0, -0.0, np.inf, -np.inf]),
                        # exact ties between two float16 neighbours around 1.0
                        np.float32([1 + 2 ** -11, 1 + 3 * 2 ** -11, 2048 + 1, 2048 + 3])])
    ours = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):   # 65520 and +-1e6 round to +-inf on purpose
        ref = x.astype(np.float16)
    assert np.array_equal(ours, ref.view(np.uint16))
    assert O.f32_to_f16_bits(np.float32([np.nan]))[0] & 0x7E00 == 0x7E00


def test_bf16_round_trip_rne():
    import torch  # CPU-only use: an independent RNE conversion

    rng = np.random.default_rng(4)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 1e3,
                        np.float32([1 + 2 ** -8, 1 + 3 * 2 ** -8, 0.0, -0.0, np.inf, -np.inf, 3.3895314e38])])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(x), ref)
    L = O.lib()
    for b in [0, 0x3F80, 0xC2F7, 0x0001]:
        assert L.vmo_bf16_to_f32(b) == np.array([b << 16], np.uint32).view(np.float32)[0]


def test_mixed_dtype_scalar_reference():
    # quantized_matmul.cpp:363-367: F16/BF16 activations, F16/BF16/F32 scales.
    rng = np.random.default_rng(8)
    m, k, n = 2, 64, 16
    q, s = O.quantize_int8((rng.standard_normal((k, n)) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    a16 = a.astype(np.float16)
    s16 = s.astype(np.float16)
    out = O.qmm_mixed(a16.view(np.uint16), O.F16, q, s16.view(np.uint16), O.F16, O.F16, k, O.QUANT_INT8, 0)
    ref = (a16.astype(np.float64) @ q.astype(np.float64)) * s16.astype(np.float64)
    got = out.view(np.float16).astype(np.float64)
    assert np.abs(got - ref).max() <= 2e-3 * np.abs(ref).max()
