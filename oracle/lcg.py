"""LCG test data and the sampled-dump protocol (test infrastructure; see oracle/__init__.py).

Restates runtime/sh_test.inc.c:2-25 and softhier_mlir/testing/lcg.py:13-106 of the reference:
  state0 = seed ^ 0x9E3779B9; state <- state * 1664525 + 1013904223 (mod 2^32); output = state >> 8.
  fill_fp16: element n (row-major) = fp16(float32(lo + out_{n+1} % (hi - lo + 1)) * float32(scale)), RNE.
  sample positions: pairs (out_{2n+1} % rows, out_{2n+2} % cols).
  sample lines: "<tag> r c hhhh" (fp16 code in hex).
"""
from __future__ import annotations

import re

import numpy as np

A, C, MASK = 1664525, 1013904223, 0xFFFFFFFF
SEED_MIX = 0x9E3779B9


def states_scalar(seed: int, n: int) -> np.ndarray:
    """The first n LCG states after seeding, by the plain sequential loop (sh_test.inc.c:2)."""
    s = (seed ^ SEED_MIX) & MASK
    out = np.empty(n, dtype=np.uint32)
    for i in range(n):
        s = (s * A + C) & MASK
        out[i] = s
    return out


def _affine_power(k: int) -> tuple[int, int]:
    """(a, c) with state_{i+k} = a * state_i + c (mod 2^32)."""
    ra, rc, ba, bc = 1, 0, A, C
    while k:
        if k & 1:
            ra, rc = (ba * ra) & MASK, (ba * rc + bc) & MASK
        ba, bc = (ba * ba) & MASK, (ba * bc + bc) & MASK
        k >>= 1
    return ra, rc


def states(seed: int, n: int, lanes: int = 8192) -> np.ndarray:
    """Same as states_scalar, vectorised: `lanes` sequential states, then whole rows advanced by the
    lanes-fold composed step (wrapping uint32 arithmetic)."""
    if n <= lanes:
        return states_scalar(seed, n)
    first = states_scalar(seed, lanes)
    rows = -(-n // lanes)
    a, c = _affine_power(lanes)
    out = np.empty((rows, lanes), dtype=np.uint32)
    out[0] = first
    a32, c32 = np.uint32(a), np.uint32(c)
    with np.errstate(over="ignore"):
        for r in range(1, rows):
            out[r] = out[r - 1] * a32 + c32
    return out.reshape(-1)[:n]


def stream(seed: int, n: int) -> np.ndarray:
    """n successive LCG outputs (state >> 8)."""
    return states(seed, n) >> np.uint32(8)


def fill_fp16(rows: int, cols: int, seed: int, lo: int, hi: int, scale: float = 1.0) -> np.ndarray:
    """sh_test_fill_fp16 (sh_test.inc.c:4-14): integers in [lo, hi] times scale, rounded to fp16."""
    v = stream(seed, rows * cols) % np.uint32(hi - lo + 1)
    vals = (v.astype(np.int64) + lo).astype(np.float32) * np.float32(scale)
    return vals.astype(np.float16).reshape(rows, cols)


def const_fp16(rows: int, cols: int, bits: int) -> np.ndarray:
    """sh_test_fill_const_fp16: every element is the fp16 code `bits`."""
    return np.full((rows, cols), bits & 0xFFFF, dtype=np.uint16).view(np.float16)


def col_parity_fp16(rows: int, cols: int, even_bits: int, odd_bits: int) -> np.ndarray:
    """sh_test_fill_colparity_fp16: even columns `even_bits`, odd columns `odd_bits`."""
    row = np.where(np.arange(cols) % 2 == 1, odd_bits & 0xFFFF, even_bits & 0xFFFF).astype(np.uint16)
    return np.tile(row, (rows, 1)).view(np.float16)


def sample_positions(rows: int, cols: int, seed: int, nsamples: int) -> list[tuple[int, int]]:
    """The (i, j) sequence of sh_test_dump_samples (sh_test.inc.c:18-25)."""
    v = stream(seed, 2 * nsamples)
    return [(int(v[2 * n]) % rows, int(v[2 * n + 1]) % cols) for n in range(nsamples)]


def check_gemm_positions(M: int, N: int, nsamples: int) -> list[tuple[int, int]]:
    """The (i, j) sequence of sh_test_check_gemm (sh_test.inc.c:33-39): seed state 0xC0FFEE (no mixing),
    i = (n * 7919 + out) % M, j = (n * 104729 + out') % N in uint32 arithmetic."""
    s = 0xC0FFEE
    out = []
    for n in range(nsamples):
        s = (s * A + C) & MASK
        i = ((n * 7919 + (s >> 8)) & MASK) % M
        s = (s * A + C) & MASK
        j = ((n * 104729 + (s >> 8)) & MASK) % N
        out.append((i, j))
    return out


_SAMPLE_RE = re.compile(r"^(\S+) (\d+) (\d+) ([0-9a-fA-F]{4})$")


def parse_samples(text: str) -> dict[str, list[tuple[int, int, float]]]:
    """'<tag> r c hex' lines -> {tag: [(r, c, value)]} (lcg.py:79-90)."""
    out: dict[str, list[tuple[int, int, float]]] = {}
    for ln in text.splitlines():
        m = _SAMPLE_RE.match(ln.strip())
        if m:
            val = np.array([int(m.group(4), 16)], dtype=np.uint16).view(np.float16)[0]
            out.setdefault(m.group(1), []).append((int(m.group(2)), int(m.group(3)), float(val)))
    return out


def compare_samples(samples, ref: np.ndarray, atol: float, rtol: float) -> tuple[int, float]:
    """(mismatches, max abs error) with |got - want| <= atol + rtol |want| (lcg.py:93-106)."""
    bad, maxerr = 0, 0.0
    for r, c, got in samples:
        want = float(ref[r, c])
        err = abs(got - want)
        maxerr = max(maxerr, err)
        if err > atol + rtol * abs(want):
            bad += 1
    return bad, maxerr
