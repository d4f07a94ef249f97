"""ctypes wrapper of oracle/liboracle.so (the plain-C restatement; test infrastructure only)."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        P = C.c_void_p
        u32, u64, f32 = C.c_uint32, C.c_uint64, C.c_float
        sigs = {
            "oc_h2f": (f32, [C.c_uint16]), "oc_f2h": (C.c_uint16, [f32]),
            "oc_f2h_array": (None, [P, P, u64]), "oc_h2f_array": (None, [P, P, u64]),
            "oc_fill_fp16": (None, [P, u32, u32, u32, C.c_int, C.c_int, f32]),
            "oc_sample_positions": (None, [P, u32, u32, u32, u32]),
            "oc_gemm": (None, [P, P, P, u32, u32, u32]),
            "oc_layernorm": (None, [P, P, P, P, u32, u32, f32]),
            "oc_softmax": (None, [P, P, u32, u32, f32]),
            "oc_gelu": (None, [P, P, u64]),
            "oc_attention": (None, [P, P, P, P, u32, u32, u32, f32]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(_lib, name)
            fn.restype, fn.argtypes = res, args
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def f2h(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    load().oc_f2h_array(_p(x), _p(out), x.size)
    return out


def h2f(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    load().oc_h2f_array(_p(h), _p(out), h.size)
    return out


def fill_fp16(rows, cols, seed, lo, hi, scale=1.0) -> np.ndarray:
    out = np.empty((rows, cols), np.uint16)
    load().oc_fill_fp16(_p(out), rows, cols, seed, lo, hi, scale)
    return out.view(np.float16)


def sample_positions(rows, cols, seed, n) -> list[tuple[int, int]]:
    pos = np.empty(2 * n, np.uint32)
    load().oc_sample_positions(_p(pos), rows, cols, seed, n)
    return [(int(pos[2 * i]), int(pos[2 * i + 1])) for i in range(n)]


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float16)).view(np.uint16)


def gemm(x, w) -> np.ndarray:
    x, w = _u16(x), _u16(w)
    M, K = x.shape
    N = w.shape[1]
    z = np.empty((M, N), np.float32)
    load().oc_gemm(_p(x), _p(w), _p(z), M, N, K)
    return z


def layernorm(x, g, b, eps) -> np.ndarray:
    x, g, b = _u16(x), _u16(g), _u16(b)
    y = np.empty(x.shape, np.float32)
    load().oc_layernorm(_p(x), _p(g), _p(b), _p(y), x.shape[0], x.shape[1], eps)
    return y


def softmax(x, scale) -> np.ndarray:
    x = _u16(x)
    y = np.empty(x.shape, np.float32)
    load().oc_softmax(_p(x), _p(y), x.shape[0], x.shape[1], scale)
    return y


def gelu(x) -> np.ndarray:
    x = _u16(x)
    y = np.empty(x.shape, np.float32)
    load().oc_gelu(_p(x), _p(y), x.size)
    return y


def attention(q, k, v, heads, scale) -> np.ndarray:
    q, k, v = _u16(q), _u16(k), _u16(v)
    S, D = q.shape
    o = np.empty((S, D), np.uint16)
    load().oc_attention(_p(q), _p(k), _p(v), _p(o), S, D, heads, scale)
    return o.view(np.float16)
