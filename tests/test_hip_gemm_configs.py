"""Every MFMA GEMM tile variant (rows_m > 4), forced through the tuning
overrides (VELOMIND_GEMM_CFG="BM,BN,S[,D]" for the small-tile kernel,
VELOMIND_GEMM_WIDE="BM,BN,S,D,G" for the wide one), against the oracle.

Per-column INT8 takes either kernel; blockwise weights (INT4, INT8 with
blocks) always take the wide kernel, which multiplies each 32-row chunk's
fp32 sum by its block scale (codes exact in fp16), in its tile shapes with
two 32 x 32 tiles per wave.  Covers K splits 1/2/4 (deterministic split-K
reduction), partial M and N tiles, K ending half-way through a 64-row step,
INT8 blocks of 32 and 96 rows, and block scales from 1e-7 to 1e3.  Bound:
the north-star 1e-3 * max|ref|; test_activation_magnitudes also holds every
kind to fp32 summation bounds against the reference loop.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

# (BM, BN) tile variants instantiated in velo-mind_amd/csrc/qmm_gemm.hip.
TILES = [(16, 128), (32, 128), (64, 128), (128, 128), (16, 64), (32, 64), (64, 64)]
TOL = 1e-3


def _check(out, ref, tol=TOL):
    ref = np.asarray(ref, np.float64)
    err = np.abs(out.astype(np.float64) - ref).max()
    bound = tol * max(np.abs(ref).max(), 1e-30)
    assert err <= bound, f"max abs err {err:.3e} > {bound:.3e}"


def _weights(kind, k, n, rng, block):
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    if kind == "int8":
        q, s = O.quantize_int8(w)
        return q, s, 1, 0
    if kind == "int8_block":
        q = rng.integers(-127, 128, (k, n), dtype=np.int8)
        s = (rng.random(((k + block - 1) // block, n)) * 0.01 + 1e-4).astype(np.float32)
        return q, s, 1, block
    q, s = O.quantize_int4(w, block)
    return q, s, 2, block


@pytest.mark.parametrize("kind,block", [("int8", 0)])
@pytest.mark.parametrize("bm,bn", TILES)
def test_forced_tile(hip, monkeypatch, bm, bn, kind, block):
    m, k, n = 40, 224, 336        # partial M and N tiles; 224 = 3.5 steps of 64
    rng = np.random.default_rng(bm * 1000 + bn + block)
    q, s, qt, blk = _weights(kind, k, n, rng, block)
    oq = O.QUANT_INT4 if qt == 2 else O.QUANT_INT8
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.qmm(x, q.view(np.int8), s, k, oq, blk)
    for splits in (1, 2, 4):
        monkeypatch.setenv("VELOMIND_GEMM_CFG", f"{bm},{bn},{splits}")
        print(f"case BM={bm} BN={bn} S={splits} kind={kind} block={block} m={m} k={k} n={n}", flush=True)
        out = hip.run_qmm(x, q, s, k, qt, blk)
        _check(out, ref)
    monkeypatch.delenv("VELOMIND_GEMM_CFG")


@pytest.mark.parametrize("kind,block", [("int8", 0)])
@pytest.mark.parametrize("bm,deep", [(16, 4), (16, 8), (32, 4), (32, 8)])
@pytest.mark.parametrize("m", [5, 16, 40])
def test_forced_deep(hip, monkeypatch, bm, deep, kind, block, m):
    # K = 992 rows = 15.5 steps of 64: with D steps in flight the split
    # count is at least ceil(16 / D), and the last split is partial (its
    # trailing steps read zeros); N = 336 leaves a partial column tile.
    k, n = 992, 336
    rng = np.random.default_rng(bm * 100 + deep * 10 + m + block)
    q, s, qt, blk = _weights(kind, k, n, rng, block)
    oq = O.QUANT_INT4 if qt == 2 else O.QUANT_INT8
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.qmm(x, q.view(np.int8), s, k, oq, blk)
    steps = (k + 63) // 64
    for splits in sorted({-(-steps // deep), -(-steps // deep) + 1, 16}):
        monkeypatch.setenv("VELOMIND_GEMM_CFG", f"{bm},64,{splits},{deep}")
        print(f"case BM={bm} D={deep} S={splits} kind={kind} block={block} m={m} k={k} n={n}", flush=True)
        out = hip.run_qmm(x, q, s, k, qt, blk)
        _check(out, ref)
    monkeypatch.delenv("VELOMIND_GEMM_CFG")


@pytest.mark.parametrize("mag", [1e-7, 1e-3, 1e3])
@pytest.mark.parametrize("qt", ["int4", "int8_block"])
def test_scale_magnitudes(hip, mag, qt):
    # Block scales spanning 3 orders of magnitude inside each column.
    m, k, n, block = 33, 256, 128, 32
    rng = np.random.default_rng(int(mag * 1e7) % 1000 + 3)
    nb = k // block
    spread = 10.0 ** rng.uniform(-1.5, 1.5, (nb, n))
    s = (mag * spread).astype(np.float32)
    if qt == "int4":
        codes = rng.integers(-8, 8, (k, n))
        packed = np.zeros(((k + 1) // 2, n), np.uint8)
        packed |= (codes[0::2] & 0xF).astype(np.uint8)
        packed |= ((codes[1::2] & 0xF) << 4).astype(np.uint8)
        q, hq, oq = packed, hip.QUANT_INT4, O.QUANT_INT4
    else:
        q, hq, oq = rng.integers(-127, 128, (k, n), dtype=np.int8), hip.QUANT_INT8, O.QUANT_INT8
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.qmm(x, q.view(np.int8), s, k, oq, block)
    out = hip.run_qmm(x, q, s, k, hq, block)
    # columns differ by orders of magnitude: hold each column to its own max
    ref64 = np.asarray(ref, np.float64)
    colmax = np.abs(ref64).max(axis=0)
    err = np.abs(out.astype(np.float64) - ref64).max(axis=0)
    assert np.all(err <= TOL * np.maximum(colmax, 1e-300)), f"worst column ratio {np.max(err / colmax):.3e}"


def test_split_k_deterministic(hip, monkeypatch):
    m, k, n = 24, 2048, 640
    rng = np.random.default_rng(5)
    q, s = O.quantize_int4((rng.standard_normal((k, n)) * 0.02).astype(np.float32), 32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    monkeypatch.setenv("VELOMIND_GEMM_WIDE", "64,128,8,2,1")   # eight K splits of the blockwise kernel
    outs = [hip.run_qmm(x, q, s, k, hip.QUANT_INT4, 32) for _ in range(3)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    _check(outs[0], O.qmm(x, q.view(np.int8), s, k, O.QUANT_INT4, 32))


def _magnitude_rows(rng, k):
    """Rows of A at |a| ~ 1e-6, 1, 1e5, 1e6 and 1e30, and one row whose
    entries span 1e-6 .. 1e6 (the MFMA path stages each row with its own
    power-of-two scale, split into two fp16 parts)."""
    base = rng.standard_normal((6, k)).astype(np.float32)
    mags = np.array([1e-6, 1.0, 1e5, 1e6, 1e30], np.float32)
    x = base.copy()
    x[:5] *= mags[:, None]
    x[5] *= (10.0 ** rng.uniform(-6, 6, k)).astype(np.float32)
    return x


@pytest.mark.parametrize("kind,block", [("int8", 0), ("int8_block", 32), ("int4", 32)])
@pytest.mark.parametrize("reps", [1, 8, 30])      # m = 6, 48, 180: DEEP, small-M and large-M tiles
def test_activation_magnitudes(hip, kind, block, reps):
    import llama_oracle as LO

    k, n = 256, 320
    rng = np.random.default_rng(17 + reps)
    q, s, qt, blk = _weights(kind, k, n, rng, block)
    oq = O.QUANT_INT4 if qt == 2 else O.QUANT_INT8
    x = np.tile(_magnitude_rows(rng, k), (reps, 1))
    print(f"case magnitudes kind={kind} m={x.shape[0]} k={k} n={n}", flush=True)
    out = hip.run_qmm(x, q, s, k, qt, blk).astype(np.float64)
    assert np.isfinite(out).all()
    ref = np.asarray(O.qmm(x, q.view(np.int8), s, k, oq, blk), np.float64)
    rowmax = np.abs(ref).max(axis=1)
    err = np.abs(out - ref).max(axis=1)
    assert np.all(err <= TOL * rowmax), f"worst row ratio {np.max(err / rowmax):.3e}"
    # Against the model of what the MFMAs multiply (A split into two fp16
    # parts, the exact weights) the only difference left is fp32 summation
    # of 2k products and the chunk sums' scaling: |err| <= 2k * 2^-24 *
    # sum_k |a * w|.
    lin = LO.Linear(q=q, s=s, k=k, n=n, quant_type=oq, block=blk, mode=LO.LINEAR_DENSE)
    wd = lin.dense().astype(np.float64)
    model = LO.split_rows_fp16(x) @ wd
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd)
    bound = 2 * k * 2.0 ** -24 * 1.01 * mag + 1e-300
    assert np.all(np.abs(out - model) <= bound), f"worst ratio {np.max(np.abs(out - model) / bound):.3e}"
    # every kind is fp32-equivalent against the reference loop itself
    bound = (2.0 ** -22 + 4 * k * 2.0 ** -24) * 1.01 * mag + 1e-300
    assert np.all(np.abs(out - ref) <= bound), f"worst ratio {np.max(np.abs(out - ref) / bound):.3e}"


# Wide-tile variants, forced through VELOMIND_GEMM_WIDE="BM,BN,S,D,G": per-column
# INT8 takes all of them, blockwise weights the ones with two 32 x 32 tiles per wave.
WIDE_INT8 = [(128, 128, 2, 1), (128, 128, 2, 2), (128, 128, 4, 1), (64, 128, 2, 1), (64, 128, 4, 1), (128, 64, 2, 1),
             (128, 64, 2, 2), (64, 256, 2, 1)]
WIDE_BLOCK = [(128, 64, 2, 1), (128, 64, 2, 2), (64, 128, 2, 1)]
WIDE_CASES = ([("int8", 0) + t for t in WIDE_INT8] +
              [kb + t for kb in (("int8_block", 32), ("int8_block", 96), ("int4", 32), ("int4", 64)) for t in WIDE_BLOCK])


@pytest.mark.parametrize("kind,block,bm,bn,depth,groups", WIDE_CASES)
@pytest.mark.parametrize("m", [6, 40, 130])
def test_forced_wide(hip, monkeypatch, bm, bn, depth, groups, kind, block, m):
    # K = 224 = 3.5 steps of 64; N = 336 leaves partial tiles for every BN;
    # m = 130 leaves a 2-row M tile after 128.
    k, n = 224, 336
    rng = np.random.default_rng(bm * 7 + bn + depth * 3 + groups * 5 + block + m)
    q, s, qt, blk = _weights(kind, k, n, rng, block)
    oq = O.QUANT_INT4 if qt == 2 else O.QUANT_INT8
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.qmm(x, q.view(np.int8), s, k, oq, blk)
    for splits in (1, 2, 4):
        monkeypatch.setenv("VELOMIND_GEMM_WIDE", f"{bm},{bn},{splits},{depth},{groups}")
        print(f"case wide BM={bm} BN={bn} D={depth} G={groups} S={splits} kind={kind} block={block} m={m} k={k} n={n}",
              flush=True)
        out = hip.run_qmm(x, q, s, k, qt, blk)
        _check(out, ref)
    monkeypatch.delenv("VELOMIND_GEMM_WIDE")


@pytest.mark.parametrize("kind,block", [("int8", 0), ("int4", 32)])
def test_wide_long_k(hip, monkeypatch, kind, block):
    # K = 2048: every ring stage wraps several times; the default rule's splits
    m, k, n = 200, 2048, 512
    rng = np.random.default_rng(91 + block)
    q, s, qt, blk = _weights(kind, k, n, rng, block)
    oq = O.QUANT_INT4 if qt == 2 else O.QUANT_INT8
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.qmm(x, q.view(np.int8), s, k, oq, blk)
    print(f"case wide long-k default kind={kind} m={m} k={k} n={n}", flush=True)
    _check(hip.run_qmm(x, q, s, k, qt, blk), ref)
    forced = "128,128,3,2,2" if kind == "int8" else "128,64,3,2,2"
    monkeypatch.setenv("VELOMIND_GEMM_WIDE", forced)
    print(f"case wide long-k {forced} kind={kind}", flush=True)
    _check(hip.run_qmm(x, q, s, k, qt, blk), ref)
    monkeypatch.delenv("VELOMIND_GEMM_WIDE")
