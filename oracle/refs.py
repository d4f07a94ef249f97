"""numpy reference results of the hot-path ops (test infrastructure; see oracle/__init__.py).

All math is fp32 on fp16 inputs; `r16` marks where the reference device stores an fp16 intermediate.
Sources (runwangdl/softhier-mlir):
  gemm       tests/gvsoc/run.py:116-121   z = x.astype(f32) @ w.astype(f32) (+ z0), compared in fp32
  row ops    tests/gvsoc/run.py:152-158   LN (biased var, eps inside sqrt), softmax(scale x) with max
             subtraction, tanh-GELU, add, add_bias (per column), scale, transpose; siglip_ref.py:20-22, 42
  attention  tests/gvsoc/run.py:921-934   s = r16(q k^T) * scale; p = r16(softmax(s)); o = r16(p v)
  encoder    softhier_mlir/testing/siglip_ref.py:9-45 with the op order of frontend/siglip.py:133-168
  llm ops    tests/gvsoc/run.py:175-235   RMSNorm, RoPE (rotate-half), silu(a) b, token-masked softmax, GQA
             attention (semantics of runtime/sh_ops.h:277-304)
"""
from __future__ import annotations

import numpy as np

from oracle import lcg

F32 = np.float32


def r16(a: np.ndarray) -> np.ndarray:
    """Round to fp16 and back (a stored fp16 intermediate)."""
    return np.asarray(a, dtype=F32).astype(np.float16).astype(F32)


def f32(a) -> np.ndarray:
    return np.asarray(a).astype(F32)


# ---- GEMM -----------------------------------------------------------------------------------------------
def gemm(x: np.ndarray, w: np.ndarray, z0: np.ndarray | None = None) -> np.ndarray:
    """fp32 X @ W (+ Z0), unrounded (run.py:118)."""
    z = f32(x) @ f32(w)
    return z if z0 is None else z + f32(z0)


# ---- row ops --------------------------------------------------------------------------------------------
def layernorm(x, g, b, eps: float) -> np.ndarray:
    x = f32(x)
    m = x.mean(1, keepdims=True)
    v = x.var(1, keepdims=True)
    return (x - m) / np.sqrt(v + F32(eps)) * f32(g) + f32(b)


def softmax(x, scale: float) -> np.ndarray:
    t = F32(scale) * f32(x)
    e = np.exp(t - t.max(1, keepdims=True))
    return e / e.sum(1, keepdims=True)


def gelu(x) -> np.ndarray:
    x = f32(x)
    return F32(0.5) * x * (F32(1) + np.tanh(F32(0.7978845608) * (x + F32(0.044715) * x ** 3)))


def add(a, b) -> np.ndarray:
    return f32(a) + f32(b)


def add_bias(x, bias_row) -> np.ndarray:
    return f32(x) + f32(bias_row).reshape(1, -1)


def scale(x, s: float) -> np.ndarray:
    return f32(x) * F32(s)


def transpose(x: np.ndarray) -> np.ndarray:
    """Bit-exact: pure data movement (works on any dtype, including uint16 fp16 codes)."""
    return np.ascontiguousarray(np.asarray(x).T)


# ---- attention ------------------------------------------------------------------------------------------
def attention(q, k, v, heads: int, scale: float = 0.125) -> np.ndarray:
    """One sequence, [S, D] operands, head h = columns [h dh, (h+1) dh) (run.py:921-934)."""
    q, k, v = f32(q), f32(k), f32(v)
    S, D = q.shape
    dh = D // heads
    o = np.zeros((S, D), F32)
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        s = r16(q[:, sl] @ k[:, sl].T) * F32(scale)
        p = np.exp(s - s.max(1, keepdims=True))
        p = r16(p / p.sum(1, keepdims=True))
        o[:, sl] = r16(p @ v[:, sl])
    return o


def attention_batched(q, k, v, B: int, heads: int, scale: float = 0.125) -> np.ndarray:
    """[B*S, D] operands, sequence b = rows [b S, (b+1) S)."""
    S = q.shape[0] // B
    return np.concatenate([attention(q[b * S:(b + 1) * S], k[b * S:(b + 1) * S], v[b * S:(b + 1) * S], heads, scale)
                           for b in range(B)], axis=0)


def attention_reference_lcg(S: int, D: int, H: int, scale: float = 0.125) -> np.ndarray:
    """run.py:921-934 on the reference's LCG inputs (seeds 21 / 22 / 23)."""
    q = lcg.fill_fp16(S, D, 21, -8, 8, 0.125)
    k = lcg.fill_fp16(S, D, 22, -8, 8, 0.125)
    v = lcg.fill_fp16(S, D, 23, -16, 16, 0.125)
    return attention(q, k, v, H, scale)


# ---- encoder layer --------------------------------------------------------------------------------------
PARAM_NAMES = ("wq", "wk", "wv", "wo", "w1", "w2", "bq", "bk", "bv", "bo", "b1", "b2", "g1", "be1", "g2", "be2")


def encoder_layer(x, p: dict, heads: int, B: int = 1, eps: float = 1e-6, keep: bool = False) -> dict | np.ndarray:
    """One pre-LN SigLIP layer on [B*S, D] rows with fp16 rounding at each stored intermediate
    (siglip_ref.py:24-45; op order siglip.py:133-168). Returns OUT, or every intermediate when keep=True."""
    x = f32(x)
    ln1 = r16(layernorm(x, p["g1"], p["be1"], eps))
    q = r16(r16(ln1 @ f32(p["wq"])) + f32(p["bq"]))
    k = r16(r16(ln1 @ f32(p["wk"])) + f32(p["bk"]))
    v = r16(r16(ln1 @ f32(p["wv"])) + f32(p["bv"]))
    o = attention_batched(q, k, v, B, heads, 1.0 / np.sqrt(x.shape[1] // heads))
    ao = r16(r16(o @ f32(p["wo"])) + f32(p["bo"]))
    h = r16(x + ao)
    ln2 = r16(layernorm(h, p["g2"], p["be2"], eps))
    f1 = r16(r16(ln2 @ f32(p["w1"])) + f32(p["b1"]))
    g = r16(gelu(f1))
    f2 = r16(r16(g @ f32(p["w2"])) + f32(p["b2"]))
    out = r16(h + f2)
    if keep:
        return {"X": x, "LN1": ln1, "Q": q, "K": k, "V": v, "O": o, "AO": ao, "H": h, "LN2": ln2, "F1": f1, "G": g, "F2": f2,
                "OUT": out}
    return out


def siglip_params_lcg(D: int, F: int, layer: int = 0) -> dict:
    """The reference's LCG parameter table (siglip_ref.py:12-18, siglip.py:110-124: layer L adds 100 L)."""
    s0 = 100 * layer
    f = lcg.fill_fp16
    p = {nm: f(D, D, sd + s0, -8, 8, 1 / 128) for nm, sd in (("wq", 2), ("wk", 3), ("wv", 4), ("wo", 5))}
    p["w1"] = f(D, F, 6 + s0, -8, 8, 1 / 128)
    p["w2"] = f(F, D, 7 + s0, -8, 8, 1 / 256)
    for nm, sd in (("bq", 8), ("bk", 9), ("bv", 10), ("bo", 11)):
        p[nm] = f(1, D, sd + s0, -4, 4, 0.0625)
    p["b1"] = f(1, F, 12 + s0, -4, 4, 0.0625)
    p["b2"] = f(1, D, 13 + s0, -4, 4, 0.0625)
    p["g1"] = f(1, D, 14 + s0, 2, 6, 0.25)
    p["be1"] = f(1, D, 15 + s0, -4, 4, 0.125)
    p["g2"] = f(1, D, 16 + s0, 2, 6, 0.25)
    p["be2"] = f(1, D, 17 + s0, -4, 4, 0.125)
    return p


def siglip_input_lcg(S: int, D: int) -> np.ndarray:
    return lcg.fill_fp16(S, D, 1, -16, 16, 0.125)


def encoder_stack(x, params: list[dict], heads: int, B: int = 1, eps: float = 1e-6) -> np.ndarray:
    """`len(params)` layers, each reading the previous layer's output (siglip.py:168)."""
    for p in params:
        x = encoder_layer(x, p, heads, B, eps)
    return x


# ---- tolerance ------------------------------------------------------------------------------------------
# ---- Llama-style decoder ops (run.py:175-235; sh_ops.h:277-304) ----------------------------------------
LLM_PAD = 0xFFFF


def rmsnorm(x, g, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * g per row (run.py:232, HF LlamaRMSNorm; fp32 statistics)."""
    x = f32(x)
    return x / np.sqrt((x * x).mean(1, keepdims=True) + eps) * f32(g)


def rope(x, table, dh: int) -> np.ndarray:
    """HF rotate-half RoPE on every dh-wide head of each row (run.py:233-234): table row = cos[dh/2] | sin[dh/2]
    for that row's position; y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin."""
    x, t = f32(x), f32(table)
    S, D = x.shape
    xh = x.reshape(S, D // dh, dh)
    x1, x2 = xh[..., :dh // 2], xh[..., dh // 2:]
    c, s = t[:, None, :dh // 2], t[:, None, dh // 2:dh]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1).reshape(S, D)


def silu_mul(a, b) -> np.ndarray:
    """silu(a) * b = a / (1 + e^-a) * b (run.py:235)."""
    a = f32(a)
    return a / (1 + np.exp(-a)) * f32(b)


def llm_tokens(S: int, kind: str) -> np.ndarray:
    """Token classes of the reference's llmops driver (run.py:175-183 == llmops/main.c tok_prefix): causal
    tok[j] = j; prefix: image tokens 0, the first 5 language tokens 0, the rest PAD, the state token 1."""
    if kind == "causal":
        return np.arange(S, dtype=np.uint32)
    img = S - 64
    tok = np.full(S, LLM_PAD, dtype=np.uint32)
    tok[:img] = 0
    tok[img:img + 5] = 0
    tok[img + 48] = 1
    return tok


def softmax_masked(x, scale: float, tok_q, tok_k) -> np.ndarray:
    """softmax(scale x) over the keys j with tok_k[j] <= tok_q[i] (unsigned); a PAD query row (or one with no
    allowed key) is uniform (run.py:186-196)."""
    x = f32(x)
    tq, tk = np.asarray(tok_q, np.int64), np.asarray(tok_k, np.int64)
    allowed = (tk[None, :] <= tq[:, None]) & (tq[:, None] != LLM_PAD)
    z = np.where(allowed, scale * x, -np.inf)
    m = np.where(allowed.any(1, keepdims=True), z.max(1, keepdims=True, initial=-np.inf), 0.0)
    e = np.where(allowed, np.exp(z - m), 0.0)
    s = e.sum(1, keepdims=True)
    return np.where(s > 0, e / np.where(s > 0, s, 1.0), 1.0 / x.shape[1]).astype(F32)


def attention_gqa(q, k, v, H: int, Hkv: int, tok=None, scale: float = 0.125) -> np.ndarray:
    """H query heads over Hkv key/value heads (head h reads kv head h // (H / Hkv)), optional token mask
    (run.py:199-216): s = r16(q k^T), p = masked softmax(scale s) (plain softmax without a mask), o = r16(r16(p) v)."""
    q, k, v = f32(q), f32(k), f32(v)
    S, D = q.shape
    dh, grp = D // H, H // Hkv
    o = np.zeros((S, D), F32)
    for hd in range(H):
        sl, kv = slice(hd * dh, (hd + 1) * dh), slice((hd // grp) * dh, (hd // grp + 1) * dh)
        s = r16(q[:, sl] @ k[:, kv].T)
        if tok is None:
            p = np.exp(scale * s - (scale * s).max(1, keepdims=True))
            p = p / p.sum(1, keepdims=True)
        else:
            p = softmax_masked(s, scale, tok, tok)
        o[:, sl] = r16(r16(p) @ v[:, kv])
    return o


def pixel_shuffle(src: np.ndarray, grid: int, s: int) -> np.ndarray:
    """[grid^2, D] raster patch tokens -> [(grid/s)^2, D s^2]: output token (gr, gb) = the s x s patch block at
    rows gr s.., cols gb s.., row-major (sh_ops.h:305-307, SmolVLMConnector.pixel_shuffle). Bit-exact."""
    D = src.shape[1]
    g = grid // s
    blocks = src.reshape(g, s, g, s, D).transpose(0, 2, 1, 3, 4)        # [gr, gb, i, j, D]
    return blocks.reshape(g * g, s * s * D)


def close(got, want, atol: float = 2e-2, rtol: float = 1e-2) -> tuple[int, float, float]:
    """(elements outside |got - want| <= atol + rtol |want|, max abs error, max |want|)."""
    got, want = f32(got), f32(want)
    err = np.abs(got - want)
    bad = int(np.count_nonzero(~(err <= atol + rtol * np.abs(want))))
    return bad, float(err.max(initial=0.0)), float(np.abs(want).max(initial=0.0))
