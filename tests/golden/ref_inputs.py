"""Inputs of the reference's own quantization tests, regenerated in numpy.

The reference fills weight matrices with ``std::mt19937(1337)`` fed through
libstdc++'s ``std::uniform_real_distribution<float>(lo, hi)``
(tests/test_quantization.cpp:37-45) and activations with
``0.05f * ((i % 23) - 11)`` (tests/test_quantization.cpp:47-53).

libstdc++ maps one 32-bit draw ``u`` to ``canon = float(u) / 2**32`` (one
draw suffices for a 24-bit float mantissa; a result of 1.0 is replaced by
the float just below it) and returns ``canon * (hi - lo) + lo`` evaluated in
float.  ``mt19937_uniform_fixture.json`` (written by
``gen_mt19937_fixture.cpp`` with the system libstdc++) pins this
regeneration bit for bit.
"""
from __future__ import annotations

import numpy as np


def mt19937_u32(seed: int, count: int) -> np.ndarray:
    """First ``count`` outputs of std::mt19937(seed) (init_genrand seeding)."""
    bitgen = np.random.MT19937()
    bitgen._legacy_seeding(seed)
    return bitgen.random_raw(count).astype(np.uint32)


def uniform_float(seed: int, count: int, lo: float, hi: float) -> np.ndarray:
    u = mt19937_u32(seed, count)
    canon = u.astype(np.float32) / np.float32(4294967296.0)
    below_one = np.nextafter(np.float32(1.0), np.float32(0.0))
    canon = np.where(canon >= np.float32(1.0), below_one, canon).astype(np.float32)
    span = np.float32(hi) - np.float32(lo)
    return (canon * span + np.float32(lo)).astype(np.float32)


def generate_random_weights(rows: int, cols: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """tests/test_quantization.cpp:37-45 (row-major [rows, cols])."""
    return uniform_float(1337, rows * cols, lo, hi).reshape(rows, cols)


def generate_activations(m: int, k: int) -> np.ndarray:
    """tests/test_quantization.cpp:47-53."""
    i = np.arange(m * k, dtype=np.int64)
    return (np.float32(0.05) * ((i % 23) - 11).astype(np.float32)).astype(np.float32).reshape(m, k)
