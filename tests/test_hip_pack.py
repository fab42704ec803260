"""GPU packers vs the oracle: codes and scales must be bit-exact
(src/quant.cpp:74-104, :125-175), at the configs' full shapes too."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import ref_inputs

pytestmark = pytest.mark.gpu


def _normal(rows, cols, seed, std=0.02):
    return (np.random.default_rng(seed).standard_normal((rows, cols)) * std).astype(np.float32)


def test_int8_kat_ties(hip):
    col = np.array([127 / 16, 0.15625, -0.15625, 0.03125, -0.03125, 0.09375, 0.0], np.float32)
    q, s = hip.run_pack_int8(col.reshape(-1, 1))
    assert s[0] == np.float32(0.0625)
    assert q[:, 0].tolist() == [127, 3, -3, 1, -1, 2, 0]


def test_int4_kat_ties_and_nibbles(hip):
    w = np.array([[7 / 16], [-0.03125], [0.15625], [0.03125]], np.float32)
    packed, s = hip.run_pack_int4(w, 4)
    assert s[0, 0] == np.float32(0.0625)
    assert packed[:, 0].tolist() == [0xF7, 0x13]


@pytest.mark.parametrize("rows,cols", [(128, 256), (576, 1536), (33, 17), (1, 5), (7, 1),
                                       # two-pass path: ragged row chunks, columns past the last
                                       # full workgroup, a single chunk, many chunks
                                       (1000, 1028), (64, 260), (4099, 2048), (97, 4096)])
def test_int8_bit_exact(hip, rows, cols):
    w = ref_inputs.generate_random_weights(rows, cols, -1.5, 1.5)
    w[:, 0] = 0.0  # an all-zero column takes scale 1.0
    q_ref, s_ref = O.quantize_int8(w)
    q, s = hip.run_pack_int8(w)
    assert np.array_equal(q, q_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols,block", [(128, 256, 32), (2048, 256, 32), (33, 17, 32), (5, 3, 2),
                                             (100, 9, 64), (64, 40, 8), (1, 4, 32)])
def test_int4_bit_exact(hip, rows, cols, block):
    w = _normal(rows, cols, rows + cols + block)
    w[:, -1] = 0.0
    p_ref, s_ref = O.quantize_int4(w, block)
    p, s = hip.run_pack_int4(w, block)
    assert np.array_equal(p, p_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


def test_pack_ties_everywhere(hip):
    # every element lands on an exact .5 after scaling (scale 1/16)
    rng = np.random.default_rng(9)
    w = (rng.integers(-254, 255, size=(64, 96)) / 32.0).astype(np.float32)
    w[0, :] = 127 / 16
    q_ref, s_ref = O.quantize_int8(w)
    q, s = hip.run_pack_int8(w)
    assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)
    w4 = (rng.integers(-14, 15, size=(64, 96)) / 32.0).astype(np.float32)
    w4[0::32, :] = 7 / 16
    p_ref, s4_ref = O.quantize_int4(w4, 32)
    p, s4 = hip.run_pack_int4(w4, 32)
    assert np.array_equal(p, p_ref) and np.array_equal(s4, s4_ref)


@pytest.mark.parametrize("k,n", [(2048, 2048), (2048, 5632), (5632, 2048), (2048, 32000)])
def test_full_size_tinyllama_int4_pack_bit_exact(hip, k, n):
    w = _normal(k, n, k * 7 + n)
    p_ref, s_ref = O.quantize_int4(w, 32)
    p, s = hip.run_pack_int4(w, 32)
    assert np.array_equal(p, p_ref)
    assert np.array_equal(s, s_ref)


def test_full_size_int8_pack_bit_exact(hip):
    w = _normal(960, 49152, 360)  # SmolLM2-360M tied lm_head shape [K, N]
    q_ref, s_ref = O.quantize_int8(w)
    q, s = hip.run_pack_int8(w)
    assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)


def test_dequant_matches_oracle(hip):
    w = _normal(70, 48, 1)
    q, s = O.quantize_int8(w)
    dq = hip.DeviceBuffer.from_array(q)
    ds = hip.DeviceBuffer.from_array(s)
    dw = hip.DeviceBuffer(w.nbytes)
    hip.dequant_int8(dq.addr, ds.addr, dw.addr, 70, 48)
    assert np.array_equal(dw.download(np.float32, w.shape), O.dequantize_int8(q, s))
    p, s4 = O.quantize_int4(w, 32)
    dp = hip.DeviceBuffer.from_array(p)
    ds4 = hip.DeviceBuffer.from_array(s4)
    hip.dequant_int4(dp.addr, ds4.addr, dw.addr, 70, 48, 32)
    assert np.array_equal(dw.download(np.float32, w.shape), O.dequantize_int4(p, s4, 70, 32))


def test_pack_rejects_odd_int4_block(hip):
    w = hip.DeviceBuffer(64)
    with pytest.raises(hip.VmHipError) as e:
        hip.pack_int4(w.addr, w.addr, w.addr, 4, 4, 3)
    assert e.value.status == hip.EINVAL and "even" in str(e.value)
