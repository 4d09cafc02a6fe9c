"""Seeded synthetic Q4_K / Q6_K tensors and activations for the tests.

Distributions follow the workload definitions: 4-bit quants uniform in [0,15],
6-bit scales/mins uniform (random bytes in the packed 12-byte field), fp16 d and
dmin drawn from |N(0, 0.02)|; Q6_K with uniform ql/qh bytes, uniform int8
scales and d from |N(0, 0.02)|; activations N(0, 1).
"""
from __future__ import annotations

import numpy as np

Q4_K, Q6_K, Q8_1 = 12, 14, 9


def q4k_blocks(rng: np.random.Generator, nblocks: int, dscale: float = 0.02) -> np.ndarray:
    b = rng.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, dscale, size=(nblocks, 2))).astype(np.float16)
    b[:, 0:4] = d.view(np.uint8).reshape(nblocks, 4)
    return b.reshape(-1)


def q6k_blocks(rng: np.random.Generator, nblocks: int, dscale: float = 0.02) -> np.ndarray:
    b = rng.integers(0, 256, size=(nblocks, 210), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, dscale, size=(nblocks, 1))).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def matrix(rng: np.random.Generator, t: int, rows: int, cols: int, dscale: float = 0.02) -> np.ndarray:
    assert cols % 256 == 0
    nb = rows * cols // 256
    return q4k_blocks(rng, nb, dscale) if t == Q4_K else q6k_blocks(rng, nb, dscale)


def representable_activation(rng: np.random.Generator, n: int) -> np.ndarray:
    """fp32 values that q8_1 holds exactly: per 32-value block an f16 scale d
    and x = d * q with integer q in [-127, 127], |q| = 127 somewhere (so the
    quantizer picks the same d back)."""
    assert n % 32 == 0
    x = np.empty(n, np.float32)
    for b in range(n // 32):
        d = np.float32(np.float16(abs(rng.normal(0.0, 1.0)) / 127.0 + 1e-3))
        q = rng.integers(-127, 128, 32)
        q[rng.integers(0, 32)] = 127 if rng.random() < 0.5 else -127
        x[32 * b:32 * b + 32] = d * q.astype(np.float32)
    return x


def activation(rng: np.random.Generator, n: int) -> np.ndarray:
    return rng.standard_normal(n).astype(np.float32)


def fixed_scale_matrix(rng: np.random.Generator, t: int, rows: int, cols: int) -> np.ndarray:
    """Random payload with every d/dmin forced to f16(0.05): the reference
    tests' fill_matrix_bytes (V/tests/test_core.c:510-542)."""
    w = matrix(rng, t, rows, cols)
    half = np.array([0.05], np.float16).view(np.uint8)
    if t == Q4_K:
        blk = w.reshape(-1, 144)
        blk[:, 0:2] = half
        blk[:, 2:4] = half
    else:
        blk = w.reshape(-1, 210)
        blk[:, 208:210] = half
    return w
