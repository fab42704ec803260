"""Every instantiated GEMV kernel shape, forced through the tuning override
(VELOMIND_GEMV_CFG="L,W,S"), against the oracle.

The automatic config rule only reaches a few (L, W, S) combinations for the
shapes of the other tests; this covers the rest: all lane widths L (16-column
groups per row segment), wave counts W, split counts S (with a partial last
split; 3 and 5 splits leave a split tree with unpaired nodes), 1/2/4 activation rows, the three weight kinds, a partial last tile and
more than eight tiles (so the XCD tile renumbering and its identity tail both
run).  Tolerance: the fp32 GEMV bound of 1e-5 * max|ref|.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

# (L, W) pairs instantiated in velo-mind_amd/csrc/qmm_gemv.hip (kShapes).
SHAPES = [(1, 4), (2, 4), (2, 8), (4, 4), (4, 8), (8, 4), (8, 8), (16, 4), (16, 8), (16, 16)]
TOL_GEMV = 1e-5


def _check(out, ref):
    ref = np.asarray(ref, np.float64)
    err = np.abs(out.astype(np.float64) - ref).max()
    bound = TOL_GEMV * max(np.abs(ref).max(), 1e-30)
    assert err <= bound, f"max abs err {err:.3e} > {bound:.3e}"


@pytest.mark.parametrize("kind", ["int8", "int8_block", "int4"])
@pytest.mark.parametrize("L,W", SHAPES)
def test_forced_config(hip, monkeypatch, L, W, kind):
    k = 1000                      # 125 chunks of 8: splits of 3 leave a short last split
    n = 16 * L * 11 - 16 * (L // 2)  # 11 tiles, the last one partial (L >= 2)
    rng = np.random.default_rng(L * 100 + W)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    if kind == "int8":
        q, s = O.quantize_int8(w)
        qt, block, oq = hip.QUANT_INT8, 0, O.QUANT_INT8
    elif kind == "int8_block":
        q = rng.integers(-127, 128, (k, n), dtype=np.int8)
        s = rng.random(((k + 31) // 32, n)).astype(np.float32) * 0.01
        qt, block, oq = hip.QUANT_INT8, 32, O.QUANT_INT8
    else:
        q, s = O.quantize_int4(w, 32)
        qt, block, oq = hip.QUANT_INT4, 32, O.QUANT_INT4
    for m in (1, 2, 4):
        x = rng.standard_normal((m, k)).astype(np.float32)
        ref = O.qmm(x, q.view(np.int8), s, k, oq, block)
        for S in (1, 3, 4, 5):
            monkeypatch.setenv("VELOMIND_GEMV_CFG", f"{L},{W},{S}")
            print(f"case L={L} W={W} S={S} kind={kind} m={m} k={k} n={n}", flush=True)
            out = hip.run_qmm(x, q, s, k, qt, block)
            _check(out, ref)
    monkeypatch.delenv("VELOMIND_GEMV_CFG")


@pytest.mark.parametrize("kind", ["int8", "int4"])
@pytest.mark.parametrize("splits", [7, 13, 31])
def test_deep_split_trees(hip, monkeypatch, kind, splits):
    """Split-K trees of up to five levels with unpaired nodes (7, 13 and 31
    splits of K = 3968, 496 chunks), one and three activation rows."""
    k, n = 3968, 256
    rng = np.random.default_rng(splits * 10 + len(kind))
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    if kind == "int8":
        q, s = O.quantize_int8(w)
        qt, block, oq = hip.QUANT_INT8, 0, O.QUANT_INT8
    else:
        q, s = O.quantize_int4(w, 32)
        qt, block, oq = hip.QUANT_INT4, 32, O.QUANT_INT4
    chunks = k // 8
    cps = -(-chunks // splits)
    assert -(-chunks // cps) == splits     # the override yields exactly this many splits
    for m in (1, 3):
        x = rng.standard_normal((m, k)).astype(np.float32)
        ref = O.qmm(x, q.view(np.int8), s, k, oq, block)
        monkeypatch.setenv("VELOMIND_GEMV_CFG", f"8,4,{splits}")
        print(f"case deep tree S={splits} kind={kind} m={m}", flush=True)
        out = hip.run_qmm(x, q, s, k, qt, block)
        again = hip.run_qmm(x, q, s, k, qt, block)
        _check(out, ref)
        assert np.array_equal(out.view(np.uint32), again.view(np.uint32))
    monkeypatch.delenv("VELOMIND_GEMV_CFG")
