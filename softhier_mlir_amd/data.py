"""Seeded synthetic inputs for the measured configurations (host-side numpy).

  - uniform(rows, cols, seed, lo, hi): the seeded 32-bit LCG of the reference's test data
    (s0 = seed ^ 0x9E3779B9, s <- 1664525 s + 1013904223 mod 2^32, v = s >> 8) mapped to
    lo + (hi - lo) (v + 0.5) / 2^24, rounded to fp16;
  - normal(shape, seed, mean, std): numpy default_rng(seed) standard normals in fp32, rounded to fp16.
"""
from __future__ import annotations

import numpy as np

_A, _C, _MASK = 1664525, 1013904223, 0xFFFFFFFF


def _lcg_states(seed: int, n: int, lanes: int = 8192) -> np.ndarray:
    s = (seed ^ 0x9E3779B9) & _MASK
    k = min(n, lanes)
    first = np.empty(k, np.uint32)
    for i in range(k):
        s = (s * _A + _C) & _MASK
        first[i] = s
    if n <= lanes:
        return first[:n]
    a, c, ba, bc = 1, 0, _A, _C          # lanes-fold step map
    m = lanes
    while m:
        if m & 1:
            a, c = (ba * a) & _MASK, (ba * c + bc) & _MASK
        ba, bc = (ba * ba) & _MASK, (ba * bc + bc) & _MASK
        m >>= 1
    rows = -(-n // lanes)
    out = np.empty((rows, lanes), np.uint32)
    out[0] = first
    with np.errstate(over="ignore"):
        for r in range(1, rows):
            out[r] = out[r - 1] * np.uint32(a) + np.uint32(c)
    return out.reshape(-1)[:n]


def uniform(rows: int, cols: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    v = (_lcg_states(seed, rows * cols) >> np.uint32(8)).astype(np.float64)
    u = (v + 0.5) / float(1 << 24)
    return (lo + (hi - lo) * u).astype(np.float32).astype(np.float16).reshape(rows, cols)


def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    g = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)
    return (g * np.float32(std) + np.float32(mean)).astype(np.float16)


def encoder_params(D: int, F: int, seed: int, w_std: float = 0.02, zero_bias: bool = True) -> dict:
    """weights N(0, 0.02), biases zero, LayerNorm gamma 1 / beta 0 (random-init SigLIP-B)."""
    shapes = {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "w1": (D, F), "w2": (F, D)}
    p = {nm: normal(shp, seed + i, 0.0, w_std) for i, (nm, shp) in enumerate(shapes.items())}
    for i, (nm, n) in enumerate((("bq", D), ("bk", D), ("bv", D), ("bo", D), ("b1", F), ("b2", D))):
        p[nm] = np.zeros((1, n), np.float16) if zero_bias else normal((1, n), seed + 10 + i, 0.0, 0.02)
    p["g1"] = np.ones((1, D), np.float16)
    p["be1"] = np.zeros((1, D), np.float16)
    p["g2"] = np.ones((1, D), np.float16)
    p["be2"] = np.zeros((1, D), np.float16)
    return p
