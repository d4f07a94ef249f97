"""Pins of the CPU oracle (oracle/): each check is chosen so a plausible slip in the restatement
(wrong constant, dropped term, transposed operand, wrong rounding point) fails at least one of them.
Runs without a GPU."""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle, lcg, refs

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_s256_d768_h12.json"


def _fixture():
    return json.loads(GOLDEN.read_text())


def _vals(samples):
    return [(r, c, float(np.array([int(h, 16)], np.uint16).view(np.float16)[0])) for r, c, h in samples]


# ---- LCG ----------------------------------------------------------------------------------------------
def test_lcg_leapfrog_equals_scalar():
    """The reference's own self-test (tests/test_testdata.py:42-45), plus block-boundary sizes."""
    for seed, n in [(1, 1), (3, 4095), (3, 4096), (3, 4097), (11, 20000), (5, 8192), (5, 8193), (7, 3 * 8192 + 5)]:
        assert np.array_equal(lcg.states(seed, n), lcg.states_scalar(seed, n))
    assert lcg.states(5, 0).shape == (0,)


def test_lcg_first_values_closed_form():
    """state1 = (seed ^ 0x9E3779B9) * 1664525 + 1013904223 mod 2^32, by Python integers."""
    for seed in (0, 1, 21, 0xFFFFFFFF):
        s1 = ((seed ^ 0x9E3779B9) * 1664525 + 1013904223) % 2**32
        s2 = (s1 * 1664525 + 1013904223) % 2**32
        assert list(lcg.states_scalar(seed, 2)) == [s1, s2]
        assert list(lcg.stream(seed, 2)) == [s1 >> 8, s2 >> 8]


def test_sample_positions_match_reference_device_log():
    """The 512 (r, c) positions the reference's device printed (seeds 301 / 302) pin the LCG end to end:
    seed mixing, constants, the >> 8 and the (row, col) order."""
    fx = _fixture()
    assert lcg.sample_positions(256, 64, 301, 256) == [(r, c) for r, c, _ in fx["samples"]["O0"]]
    assert lcg.sample_positions(256, 768, 302, 256) == [(r, c) for r, c, _ in fx["samples"]["O"]]
    assert c_oracle.sample_positions(256, 768, 302, 256) == [(r, c) for r, c, _ in fx["samples"]["O"]]


def test_fill_values_closed_form_and_c_twin():
    x = lcg.fill_fp16(9, 11, 7, -16, 16, 0.125)
    v = lcg.stream(7, 99) % 33
    assert np.array_equal(x.reshape(-1).astype(np.float32), ((v.astype(np.int64) - 16) * 0.125).astype(np.float32))
    assert np.array_equal(c_oracle.fill_fp16(37, 53, 3, -8, 8, 1 / 128).view(np.uint16),
                          lcg.fill_fp16(37, 53, 3, -8, 8, 1 / 128).view(np.uint16))
    c = lcg.fill_fp16(4, 5, 9, 3, 3)
    assert (c == 3).all()                                   # lo == hi: constant (run.py:93 Z0 = 3)
    y = lcg.fill_fp16(64, 64, 2, -2, 2)
    assert set(np.unique(y).tolist()) == {-2.0, -1.0, 0.0, 1.0, 2.0}


def test_check_gemm_positions_cover_range():
    pos = lcg.check_gemm_positions(256, 768, 256)
    assert all(0 <= i < 256 and 0 <= j < 768 for i, j in pos)
    s = 0xC0FFEE
    s = (s * 1664525 + 1013904223) % 2**32
    i0 = (s >> 8) % 256
    s = (s * 1664525 + 1013904223) % 2**32
    assert pos[0] == (i0, (s >> 8) % 768)


# ---- fp16 codec ---------------------------------------------------------------------------------------
def test_fp16_decode_exhaustive_against_numpy_and_c():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = c_oracle.h2f(h)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_fp16_encode_known_values():
    cases = {1.0: 0x3C00, -2.0: 0xC000, 65504.0: 0x7BFF, 65519.996: 0x7BFF, 65520.0: 0x7C00, 2.0 ** -24: 0x0001,
             2.0 ** -25: 0x0000, 1.5 * 2.0 ** -25: 0x0001, 2.0 ** -14: 0x0400, 1.0 + 2.0 ** -11: 0x3C00,
             1.0 + 3 * 2.0 ** -11: 0x3C02, 0.1: 0x2E66, -0.0: 0x8000, math.inf: 0x7C00}
    for f, code in cases.items():
        assert int(c_oracle.f2h(np.array([f], np.float32))[0]) == code, f
        assert int(np.array([f], np.float32).astype(np.float16).view(np.uint16)[0]) == code, f


def test_fp16_encode_random_against_numpy():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, 400_000, dtype=np.uint64).astype(np.uint32)
    u[1::2] = (u[1::2] & 0x807FFFFF) | (((u[1::2] >> 8) % 40 + 100) << 23)   # exponents around binary16's range
    u[2::8] &= ~np.uint32(0x0FFF)                                           # exact and tie patterns
    u[3::8] = (u[3::8] & ~np.uint32(0x1FFF)) | np.uint32(0x1000)
    f = u.view(np.float32)
    ok = ~np.isnan(f)
    with np.errstate(over="ignore"):
        want = f[ok].astype(np.float16).view(np.uint16)
    assert np.array_equal(c_oracle.f2h(f[ok]), want)


# ---- GEMM ---------------------------------------------------------------------------------------------
def test_gemm_small_integer_exact_and_brute_force():
    x = lcg.fill_fp16(16, 24, 1, -1, 1)
    w = lcg.fill_fp16(24, 8, 2, -2, 2)
    z = refs.gemm(x, w)
    brute = np.array([[sum(float(x[i, k]) * float(w[k, j]) for k in range(24)) for j in range(8)] for i in range(16)])
    assert np.array_equal(z, brute)                         # small integers: exact in fp32
    assert np.array_equal(z, c_oracle.gemm(x, w))
    assert not np.array_equal(refs.gemm(x[:8, :8], w[:8, :8]), refs.gemm(x[:8, :8], w[:8, :8].T))


def test_gemm_known_answers():
    x = np.ones((64, 1024), np.float16)
    w = np.full((1024, 32), 1 / 1024, np.float16)
    assert np.allclose(refs.gemm(x, w), 1.0, atol=0)        # examples/gemm1024_summa.mlir:5 (X = 1, W = 1/1024)
    z0 = lcg.fill_fp16(64, 32, 3, 3, 3)
    assert np.allclose(refs.gemm(x, w, z0), 4.0, atol=0)    # accumulate onto Z0 = 3 (run.py:93)


# ---- row ops ------------------------------------------------------------------------------------------
def test_layernorm_closed_forms():
    x = np.array([[1.0, 3.0], [-2.0, 6.0]], np.float16)
    g = np.array([[2.0, 0.5]], np.float16)
    b = np.array([[0.25, -1.0]], np.float16)
    y = refs.layernorm(x, g, b, 0.0)                        # two elements normalise to -1 / +1
    assert np.allclose(y, [[-2.0 + 0.25, 0.5 - 1.0], [-2.0 + 0.25, 0.5 - 1.0]], atol=1e-6)
    c = np.full((3, 8), 1.5, np.float16)
    assert np.allclose(refs.layernorm(c, np.ones((1, 8)), np.full((1, 8), 0.75), 1e-6), 0.75)   # constant row -> beta
    r = lcg.fill_fp16(5, 96, 11, -16, 16, 0.125)
    y = refs.layernorm(r, np.ones((1, 96)), np.zeros((1, 96)), 1e-5)
    assert np.allclose(y.mean(1), 0, atol=1e-5) and np.allclose(y.var(1), 1, atol=2e-3)       # biased variance
    gg, bb = lcg.fill_fp16(1, 96, 13, 1, 8, 0.25), lcg.fill_fp16(1, 96, 14, -4, 4, 0.25)
    assert np.allclose(refs.layernorm(r, gg, bb, 1e-5), c_oracle.layernorm(r, gg, bb, 1e-5), atol=2e-5)


def test_softmax_closed_forms():
    x = lcg.fill_fp16(7, 33, 11, -16, 16, 0.125)
    for s in (0.5, 0.125, -0.3):
        y = refs.softmax(x, s)
        assert np.allclose(y.sum(1), 1, atol=1e-6)
        assert np.allclose(refs.softmax(x.astype(np.float32) + 3.0, s), y, atol=1e-6)         # shift invariance
        assert np.allclose(y, c_oracle.softmax(x, s), atol=1e-6)
    assert np.allclose(refs.softmax(np.full((2, 10), 2.5, np.float16), 0.5), 0.1)
    two = refs.softmax(np.array([[0.0, 1.0]], np.float16), math.log(3.0))                      # e^{ln 3} : 1 = 3 : 1
    assert np.allclose(two, [[0.25, 0.75]], atol=1e-6)
    assert np.allclose(refs.softmax(x, 0.0), 1 / 33)


def test_gelu_against_erf_form():
    x = np.linspace(-6, 6, 2401, dtype=np.float32)
    erf_gelu = 0.5 * x * (1 + np.array([math.erf(v / math.sqrt(2)) for v in x], np.float32))
    assert np.abs(refs.gelu(x) - erf_gelu).max() < 1e-3      # the tanh approximation's known error bound
    assert refs.gelu(np.float32(0)) == 0
    assert abs(float(refs.gelu(np.float32(1.0))) - 0.8411919906) < 1e-6
    h = lcg.fill_fp16(3, 50, 5, -32, 32, 0.125)
    assert np.allclose(refs.gelu(h), c_oracle.gelu(h), atol=1e-6)


def test_elementwise_and_transpose():
    a = lcg.fill_fp16(4, 6, 11, -16, 16, 0.125)
    b = lcg.fill_fp16(4, 6, 12, -16, 16, 0.125)
    bias = lcg.fill_fp16(1, 6, 14, -4, 4, 0.25)
    assert np.array_equal(refs.add(a, b), a.astype(np.float32) + b.astype(np.float32))
    assert np.array_equal(refs.add_bias(a, bias)[2], a[2].astype(np.float32) + bias[0].astype(np.float32))
    assert np.array_equal(refs.scale(a, 0.3), a.astype(np.float32) * np.float32(0.3))
    codes = np.arange(4 * 6, dtype=np.uint16).reshape(4, 6) | 0x7C01      # NaN payloads survive bit-exact moves
    t = refs.transpose(codes)
    assert t.shape == (6, 4) and all(t[j, i] == codes[i, j] for i in range(4) for j in range(6))


# ---- attention ----------------------------------------------------------------------------------------
def test_attention_matches_reference_device_log():
    """All 512 logged outputs of the reference's fused attention (S=256, D=768, H=12) agree with the
    restatement within the reference's own tolerance (run.py:963), and within the north star's."""
    fx = _fixture()
    ref = refs.attention_reference_lcg(256, 768, 12)
    for tag, arr in (("O0", ref[:, :64]), ("O", ref)):
        bad, err = lcg.compare_samples(_vals(fx["samples"][tag]), arr, 0.05, 0.05)
        assert bad == 0
        bad, err = lcg.compare_samples(_vals(fx["samples"][tag]), arr, 2e-2, 1e-2)
        assert bad == 0 and err < 2e-3


def test_attention_closed_forms_and_brute_force():
    S, D, H = 16, 8, 2
    q = lcg.fill_fp16(S, D, 21, -8, 8, 0.125)
    k = lcg.fill_fp16(S, D, 22, -8, 8, 0.125)
    vrow = lcg.fill_fp16(1, D, 23, -16, 16, 0.125)
    v = np.repeat(vrow, S, 0)
    assert np.allclose(refs.attention(q, k, v, H), refs.r16(np.repeat(vrow, S, 0)), atol=2e-3)   # rows of P sum to 1
    v = lcg.fill_fp16(S, D, 23, -16, 16, 0.125)
    o0 = refs.attention(q, k, v, H, scale=0.0)                                                   # uniform weights
    assert np.allclose(o0, refs.r16(np.repeat(v.astype(np.float32).mean(0, keepdims=True), S, 0)), atol=2e-3)
    assert np.array_equal(refs.attention(q, k, v, H).view(np.uint32), refs.attention(q, k, v, H).view(np.uint32))
    assert np.allclose(refs.attention(q, k, v, H), c_oracle.attention(q, k, v, H, 0.125), atol=1e-3)
    qq, kk, vv = q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)
    o = np.zeros((S, D))
    for h in range(H):                                      # pure-Python brute force of one head at a time
        sl = slice(h * 4, h * 4 + 4)
        for i in range(S):
            s = [float(np.float16(sum(qq[i, sl][d] * kk[j, sl][d] for d in range(4)))) * 0.125 for j in range(S)]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            p = [float(np.float16(x / sum(e))) for x in e]
            for d in range(4):
                o[i, h * 4 + d] = sum(p[j] * vv[j, sl][d] for j in range(S))
    assert np.allclose(refs.attention(q, k, v, H), o, atol=1e-3)


def test_attention_batched_is_per_sequence():
    q = lcg.fill_fp16(24, 8, 1, -8, 8, 0.125)
    k = lcg.fill_fp16(24, 8, 2, -8, 8, 0.125)
    v = lcg.fill_fp16(24, 8, 3, -8, 8, 0.125)
    o = refs.attention_batched(q, k, v, 3, 2)
    assert np.array_equal(o[8:16], refs.attention(q[8:16], k[8:16], v[8:16], 2))


# ---- encoder layer ------------------------------------------------------------------------------------
def _zero_params(D, F):
    p = {nm: np.zeros(shp, np.float16) for nm, shp in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)),
                                                       ("w1", (D, F)), ("w2", (F, D)))}
    for nm, n in (("bq", D), ("bk", D), ("bv", D), ("bo", D), ("b1", F), ("b2", D), ("g1", D), ("be1", D), ("g2", D), ("be2", D)):
        p[nm] = np.zeros((1, n), np.float16)
    p["g1"][:] = 1
    p["g2"][:] = 1
    return p


def test_encoder_zero_weight_closed_form():
    """Zero weights: attention sees zero q/k/v (plus biases), so out = x + bo + gelu(b1) @ 0 + b2 = x + bo + b2."""
    D, F, S = 16, 32, 8
    p = _zero_params(D, F)
    p["bo"][:] = 0.25
    p["b2"][:] = -0.5
    x = lcg.fill_fp16(S, D, 1, -16, 16, 0.125)
    out = refs.encoder_layer(x, p, heads=2)
    assert np.allclose(out, refs.r16(refs.r16(x.astype(np.float32) + 0.25) - 0.5), atol=0)
    p["bv"][:] = 1.5                                        # V rows all 1.5 -> O = 1.5 regardless of P
    out = refs.encoder_layer(x, p, heads=2, keep=True)
    assert np.allclose(out["O"], 1.5)


def test_encoder_lcg_layer_shapes_and_composition():
    S, D, F, H = 16, 32, 64, 4
    p = refs.siglip_params_lcg(D, F)
    x = refs.siglip_input_lcg(S, D)
    r = refs.encoder_layer(x, p, H, keep=True)
    assert r["OUT"].shape == (S, D) and np.isfinite(r["OUT"]).all()
    assert np.array_equal(r["O"], refs.attention(r["Q"], r["K"], r["V"], H, 1 / math.sqrt(D // H)))
    two = refs.encoder_stack(x, [p, refs.siglip_params_lcg(D, F, 1)], H)
    assert np.array_equal(two, refs.encoder_layer(r["OUT"], refs.siglip_params_lcg(D, F, 1), H))


# (lo, hi, scale) of every tensor of the reference's LCG layer (siglip_ref.py:12-18, main.c fills)
SIGLIP_LCG_TABLE = {
    "wq": (-8, 8, 1 / 128), "wk": (-8, 8, 1 / 128), "wv": (-8, 8, 1 / 128), "wo": (-8, 8, 1 / 128),
    "w1": (-8, 8, 1 / 128), "w2": (-8, 8, 1 / 256),
    "bq": (-4, 4, 1 / 16), "bk": (-4, 4, 1 / 16), "bv": (-4, 4, 1 / 16), "bo": (-4, 4, 1 / 16),
    "b1": (-4, 4, 1 / 16), "b2": (-4, 4, 1 / 16),
    "g1": (2, 6, 1 / 4), "be1": (-4, 4, 1 / 8), "g2": (2, 6, 1 / 4), "be2": (-4, 4, 1 / 8),
}


@pytest.mark.parametrize("layer", [0, 1])
def test_siglip_lcg_params_value_sets(layer):
    """Every tensor of the LCG layer holds exactly the integers lo..hi times its scale (all of them, at the
    reference's D = 768, F = 3072), in the reference's shapes; the 16 tensors come from 16 different streams, and
    layer 1 from streams other than layer 0's. The input is {-16..16} / 8."""
    D, F = 768, 3072
    p = refs.siglip_params_lcg(D, F, layer=layer)
    shapes = {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "w1": (D, F), "w2": (F, D), "b1": (1, F)}
    for nm, (lo, hi, sc) in SIGLIP_LCG_TABLE.items():
        t = p[nm]
        assert t.dtype == np.float16 and t.shape == shapes.get(nm, (1, D)), nm
        want = {np.float16(np.float32(v) * np.float32(sc)) for v in range(lo, hi + 1)}
        assert set(np.unique(t).tolist()) == {float(v) for v in want}, nm
    heads = {nm: p[nm].ravel()[:64].tobytes() for nm in SIGLIP_LCG_TABLE}
    assert len(set(heads.values())) == len(heads)                  # no two tensors share a stream prefix
    if layer:
        p0 = refs.siglip_params_lcg(D, F, layer=0)
        assert all(not np.array_equal(p0[nm], p[nm]) for nm in SIGLIP_LCG_TABLE)
    x = refs.siglip_input_lcg(256, D)
    assert set(np.unique(x).tolist()) == {v / 8 for v in range(-16, 17)}


def test_llm_prefix_tokens_rule():
    """The prefix token classes of the reference's llmops driver (llmops/main.c tok_prefix): image tokens and the
    first 5 language tokens class 0, the state token (img + 48) class 1, every other token PAD, with
    img = S - 64; causal tokens are their own positions."""
    for S in (64, 128, 256, 1024):
        tok = refs.llm_tokens(S, "prefix")
        img = S - 64
        assert tok.shape == (S,) and tok.dtype == np.uint32
        assert (tok[:img + 5] == 0).all()
        assert tok[img + 48] == 1
        rest = np.ones(S, bool)
        rest[:img + 5] = False
        rest[img + 48] = False
        assert (tok[rest] == refs.LLM_PAD).all() and rest.sum() == 58
        assert np.array_equal(refs.llm_tokens(S, "causal"), np.arange(S))


def test_close_helper():
    bad, err, _ = refs.close(np.array([1.0, 2.0]), np.array([1.015, 2.05]))
    assert bad == 1 and abs(err - 0.05) < 1e-6


# ---- Llama-style decoder ops (run.py:175-235) ---------------------------------------------------------------
def test_rmsnorm_closed_forms():
    c = np.full((2, 8), 2.0, np.float16)
    g = lcg.fill_fp16(1, 8, 3, 1, 8, 0.25)
    y = refs.rmsnorm(c, g, 0.0)                               # constant row c: x / |c| = 1, times gamma
    assert np.allclose(y, np.repeat(g.astype(np.float32), 2, 0), atol=1e-6)
    x = lcg.fill_fp16(5, 64, 4, -16, 16, 0.125)
    y = refs.rmsnorm(x, np.ones((1, 64)), 1e-5)
    assert np.allclose(np.sqrt((y * y).mean(1)), 1, atol=1e-4)             # unit RMS
    brute = [[float(x[i, j]) / math.sqrt(sum(float(v) ** 2 for v in x[i]) / 64 + 1e-5) for j in range(64)] for i in range(5)]
    assert np.allclose(y, brute, atol=1e-5)


def test_rope_closed_forms():
    x = lcg.fill_fp16(3, 32, 5, -16, 16, 0.125)              # two heads of dh = 16
    ident = np.concatenate([np.ones((3, 8)), np.zeros((3, 8))], 1)
    assert np.array_equal(refs.rope(x, ident, 16), x.astype(np.float32))
    quarter = np.concatenate([np.zeros((3, 8)), np.ones((3, 8))], 1)       # cos 0, sin 1: (x1, x2) -> (-x2, x1)
    y = refs.rope(x, quarter, 16)
    assert np.array_equal(y[:, :8], -x[:, 8:16].astype(np.float32)) and np.array_equal(y[:, 8:16], x[:, :8].astype(np.float32))
    th = np.linspace(0, 3, 8)
    tab = np.repeat(np.concatenate([np.cos(th), np.sin(th)])[None], 3, 0)
    y = refs.rope(x, tab, 16)
    xf = x.astype(np.float64)
    for h in range(2):                                                      # rotations keep each pair's norm
        a, b = xf[:, 16 * h:16 * h + 8], xf[:, 16 * h + 8:16 * h + 16]
        ya, yb = y[:, 16 * h:16 * h + 8], y[:, 16 * h + 8:16 * h + 16]
        assert np.allclose(a * a + b * b, ya * ya + yb * yb, atol=1e-4)


def test_silu_mul_closed_forms():
    a = np.array([[0.0, 1.0, -1.0, 20.0, -20.0, 2.5]], np.float16)
    y = refs.silu_mul(a, np.ones_like(a))
    assert y[0, 0] == 0 and abs(y[0, 1] - 0.7310586) < 1e-6 and abs(y[0, 2] + 0.2689414) < 1e-6
    assert abs(y[0, 3] - 20) < 1e-6 and abs(y[0, 4]) < 1e-7
    b = lcg.fill_fp16(1, 6, 7, -4, 4, 0.5)
    assert np.allclose(refs.silu_mul(a, b), y * b.astype(np.float32), atol=1e-6)


def test_softmax_masked_closed_forms_and_brute_force():
    S = 12
    x = lcg.fill_fp16(S, S, 16, -32, 32, 0.25)
    tc = refs.llm_tokens(S, "causal")
    p = refs.softmax_masked(x, 0.5, tc, tc)
    assert np.array_equal(p[0], np.eye(S)[0]) and np.allclose(p.sum(1), 1, atol=1e-6)
    assert (np.triu(p, 1) == 0).all()                                       # nothing above the diagonal
    zeros = np.zeros(S, np.uint32)
    assert np.allclose(refs.softmax_masked(x, 0.5, zeros, zeros), refs.softmax(x, 0.5), atol=1e-6)
    tok = np.array([0, 0, 0xFFFF, 1, 0, 2, 0xFFFF, 1, 0, 0, 2, 1], np.uint32)
    p = refs.softmax_masked(x, 0.5, tok, tok)
    assert np.allclose(p[2], 1 / S) and np.allclose(p[6], 1 / S)           # padding query rows are uniform
    for i in range(S):                                                      # pure-Python brute force of the rest
        if tok[i] == 0xFFFF:
            continue
        allowed = [j for j in range(S) if tok[j] <= tok[i]]
        m = max(0.5 * float(x[i, j]) for j in allowed)
        e = {j: math.exp(0.5 * float(x[i, j]) - m) for j in allowed}
        for j in range(S):
            assert abs(p[i, j] - (e[j] / sum(e.values()) if j in e else 0.0)) < 1e-6


def test_attention_gqa_reduces_to_multi_head():
    S, H, dh = 16, 4, 8
    q = lcg.fill_fp16(S, H * dh, 21, -8, 8, 0.125)
    k = lcg.fill_fp16(S, 2 * dh, 22, -8, 8, 0.125)
    v = lcg.fill_fp16(S, 2 * dh, 23, -16, 16, 0.125)
    kk, vv = np.repeat(k.reshape(S, 2, dh), 2, 1).reshape(S, H * dh), np.repeat(v.reshape(S, 2, dh), 2, 1).reshape(S, H * dh)
    assert np.allclose(refs.attention_gqa(q, k, v, H, 2), refs.attention(q, kk, vv, H, 0.125), atol=1e-3)
    zeros = np.zeros(S, np.uint32)
    assert np.allclose(refs.attention_gqa(q, k, v, H, 2, zeros), refs.attention_gqa(q, k, v, H, 2), atol=1e-3)
    tc = refs.llm_tokens(S, "causal")
    o = refs.attention_gqa(q, k, v, H, 2, tc)
    assert np.allclose(o[0, :dh], v[0, :dh].astype(np.float32), atol=1e-3)   # query 0 sees key 0 only


def test_pixel_shuffle_brute_force():
    grid, s, D = 6, 3, 4
    src = np.arange(grid * grid * D, dtype=np.uint16).reshape(grid * grid, D)
    dst = refs.pixel_shuffle(src, grid, s)
    g = grid // s
    for gr in range(g):
        for gb in range(g):
            want = np.concatenate([src[(gr * s + i) * grid + gb * s + jj] for i in range(s) for jj in range(s)])
            assert np.array_equal(dst[gr * g + gb], want)
