"""Pins the oracle's quantize/pack/dequantize restatement (quant.cpp).

Checks, in order of strength:
  * known-answer tests built from exactly representable scales, where the
    expected codes and bytes follow from the reference's definition by hand
    (half-away-from-zero rounding, even row in the low nibble, zeroed odd-K
    high nibble, scale 1.0 for an all-zero column/block);
  * invariants that any correct implementation satisfies on random data;
  * the reference's own round-trip metric thresholds on the reference
    test's exact inputs (tests/test_quantization.cpp:100-138).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import ref_inputs


def test_int8_tie_rounds_half_away_from_zero():
    # max |x| = 127/16 -> scale = 1/16 exactly, inv = 16.
    col = np.array([127 / 16, 0.15625, -0.15625, 0.03125, -0.03125, 0.09375, 0.0], np.float32)
    q, s = O.quantize_int8(col.reshape(-1, 1))
    assert s[0] == np.float32(0.0625)
    # 2.5 -> 3 (rint would give 2), 0.5 -> 1, 1.5 -> 2.
    assert q[:, 0].tolist() == [127, 3, -3, 1, -1, 2, 0]


def test_int8_zero_column_gets_unit_scale():
    w = np.zeros((5, 3), np.float32)
    w[:, 1] = [0.5, -1.0, 0.25, 0.0, 1.0]
    q, s = O.quantize_int8(w)
    assert s[0] == 1.0 and s[2] == 1.0
    assert not q[:, 0].any() and not q[:, 2].any()
    assert s[1] == np.float32(1.0) / np.float32(127.0)
    assert q[:, 1].tolist() == [64, -127, 32, 0, 127]  # 63.5 -> 64, 31.75 -> 32


def test_int4_tie_and_nibble_order():
    # block of 4 rows, max = 7/16 -> scale = 1/16, inv = 16.
    w = np.array([[7 / 16], [-0.03125], [0.15625], [0.03125]], np.float32)
    packed, s = O.quantize_int4(w, block=4)
    assert s.shape == (1, 1) and s[0, 0] == np.float32(0.0625)
    # codes 7, -1, 3 (2.5 rounds away), 1; even row in the low nibble.
    assert packed[:, 0].tolist() == [0x7 | (0xF << 4), 0x3 | (0x1 << 4)]


def test_int4_odd_rows_leave_high_nibble_zero():
    w = np.array([[0.7, -0.7], [0.1, 0.2], [-0.35, 0.35]], np.float32)
    packed, s = O.quantize_int4(w, block=32)
    assert packed.shape == (2, 2)
    assert (packed[1] >> 4).tolist() == [0, 0]
    # row 2 is in the low nibble of packed row 1: -0.35 * 7/0.7 = -3.5 -> -4.
    assert (packed[1, 0] & 0xF) == (-4 & 0xF)
    assert (packed[1, 1] & 0xF) == 4


def test_int4_blocks_have_independent_scales():
    rows, block = 12, 4
    w = np.zeros((rows, 2), np.float32)
    w[0:4, 0] = [0.7, 0.1, 0.0, -0.2]
    w[4:8, 0] = [0.0, 0.0, 0.0, 0.0]
    w[8:12, 0] = [3.5, -7.0, 1.0, 2.0]
    w[:, 1] = np.linspace(-1, 1, rows)
    packed, s = O.quantize_int4(w, block=block)
    assert s.shape == (3, 2)
    assert s[0, 0] == np.float32(0.7) / np.float32(7)
    assert s[1, 0] == 1.0  # all-zero block
    assert s[2, 0] == np.float32(1.0)
    # block 2, column 0: codes 4 (3.5 rounds away), -7, 1, 2
    assert packed[4, 0] == ((4 & 0xF) | ((-7 & 0xF) << 4))
    assert packed[5, 0] == (1 | (2 << 4))
    assert packed[2, 0] == 0 and packed[3, 0] == 0


def _unpack_int4(packed: np.ndarray, rows: int) -> np.ndarray:
    nib = np.stack([packed & 0xF, packed >> 4], axis=1).reshape(-1, packed.shape[1])[:rows]
    return np.where(nib >= 8, nib.astype(np.int32) - 16, nib.astype(np.int32))


@pytest.mark.parametrize("rows,cols", [(64, 48), (33, 17), (1, 5), (96, 1)])
def test_int8_invariants_random(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    q, s = O.quantize_int8(w)
    amax = np.abs(w).max(axis=0)
    assert np.array_equal(s, np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32))
    assert q.min() >= -127 and q.max() <= 127
    arg = np.abs(w).argmax(axis=0)
    assert np.array_equal(np.abs(q[arg, np.arange(cols)]), np.full(cols, 127))
    err = np.abs(w.astype(np.float64) - q.astype(np.float64) * s.astype(np.float64))
    assert (err <= s.astype(np.float64) * (0.5 + 1e-5)).all()
    assert np.array_equal(O.dequantize_int8(q, s), (q.astype(np.float32) * s).astype(np.float32))


@pytest.mark.parametrize("rows,cols,block", [(64, 48, 32), (33, 17, 32), (7, 9, 2), (100, 5, 64), (1, 3, 32)])
def test_int4_invariants_random(rows, cols, block):
    rng = np.random.default_rng(rows * 7 + cols + block)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    packed, s = O.quantize_int4(w, block)
    codes = _unpack_int4(packed, rows)
    assert codes.min() >= -7 and codes.max() <= 7
    nb = (rows + block - 1) // block
    assert s.shape == (nb, cols)
    if rows % 2:
        assert not (packed[-1] >> 4).any()
    for b in range(nb):
        blk = w[b * block:(b + 1) * block]
        amax = np.abs(blk).max(axis=0)
        exp = np.where(amax > 0, amax / np.float32(7), np.float32(1)).astype(np.float32)
        assert np.array_equal(s[b], exp)
        cb = codes[b * block:(b + 1) * block]
        arg = np.abs(blk).argmax(axis=0)
        nz = amax > 0
        assert (np.abs(cb[arg, np.arange(cols)])[nz] == 7).all()
        err = np.abs(blk.astype(np.float64) - cb * s[b].astype(np.float64))
        assert (err <= s[b].astype(np.float64) * (0.5 + 1e-5)).all()
    deq = O.dequantize_int4(packed, s, rows, block)
    scale_rows = np.repeat(s, block, axis=0)[:rows]
    assert np.array_equal(deq, (codes.astype(np.float32) * scale_rows).astype(np.float32))


def test_reference_roundtrip_metrics_int8():
    # tests/test_quantization.cpp:105-118 on the reference's own inputs.
    w = ref_inputs.generate_random_weights(128, 256, -1.5, 1.5)
    q, s = O.quantize_int8(w)
    max_diff, rmse, snr, cos = O.metrics(w, O.dequantize_int8(q, s))
    assert max_diff < 0.025 and rmse < 0.01 and cos > 0.999 and snr > 40.0


def test_reference_roundtrip_metrics_int4():
    # tests/test_quantization.cpp:120-137 on the reference's own inputs.
    w = ref_inputs.generate_random_weights(128, 256, -1.5, 1.5)
    packed, s = O.quantize_int4(w, 32)
    max_diff, rmse, snr, cos = O.metrics(w, O.dequantize_int4(packed, s, 128, 32))
    assert max_diff < 0.15 and rmse < 0.08 and cos > 0.99 and snr > 20.0


def test_metrics_closed_forms():
    a = np.array([1.0, -2.0, 3.5], np.float32)
    # tests/test_quantization.cpp:420-433
    assert O.metrics(a, a) == (0.0, 0.0, 100.0, 1.0)
    md, rmse, snr, cos = O.metrics(a, 2 * a)
    assert md == pytest.approx(3.5) and rmse == pytest.approx(np.sqrt((a.astype(np.float64) ** 2).mean()))
    assert snr == pytest.approx(0.0, abs=1e-6) and cos == pytest.approx(1.0)
    md, rmse, snr, cos = O.metrics(np.array([1, 0], np.float32), np.array([0, 1], np.float32))
    assert cos == pytest.approx(0.0) and md == 1.0 and snr == pytest.approx(10 * np.log10(0.5), rel=1e-6)
    assert O.metrics(np.zeros(0, np.float32), np.zeros(0, np.float32)) == (0.0, 0.0, 0.0, 1.0)


def test_storage_sizes():
    # tests/test_quantization.cpp:376-390: INT4 packs ((K+1)/2)*N bytes.
    packed, s = O.quantize_int4(np.ones((577, 8), np.float32), 32)
    assert packed.nbytes == ((577 + 1) // 2) * 8 and s.shape == (19, 8)
