"""The Llama-style decoder ops on the GPU against the oracle (reference runtime/sh_llm.inc.c; sh_ops.h:277-307).

test_reference_llmops replays tests/gvsoc/llmops/main.c: S=256, D=960, 15 query heads over 5 key/value heads
(dh = 64), the LCG fills with its seeds, the SmolVLA-style prefix token classes and the causal ones, and the
reference's checks (run.py:219-252) at the north-star tolerance. The other tests cover the paths that driver does
not reach: widths that are not multiples of 8, the per-query attention kernel, RoPE head widths and in-place use,
the bit-exact pixel shuffle, and the argument errors the reference prints and returns on.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import _KEEP, to_dev, to_np
from oracle import lcg, refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
A = shops.addr
ALL = shops.SH_ALL


def _zeros(rows, cols):
    import torch
    return torch.zeros((rows, cols), dtype=torch.float16, device="cuda")


def _tok(arr):
    """uint16 token classes on the GPU, kept alive for the test (an inline temporary would be freed, and its
    memory handed to the next tensor, before the library's kernel reads it)."""
    import torch
    t = torch.from_numpy(np.asarray(arr, np.uint16).view(np.int16).copy()).cuda()
    _KEEP.append(t)
    return t


def test_reference_llmops(lib, gpu):
    S, D, H, Hkv, DH = 256, 960, 15, 5, 64
    DKV = Hkv * DH
    f = lambda *a: lcg.fill_fp16(*a)  # noqa: E731
    x, b, g = f(S, D, 11, -16, 16, 0.125), f(S, D, 12, -16, 16, 0.125), f(1, D, 13, 1, 8, 0.25)
    tab, sc = f(S, DH, 15, -16, 16, 0.0625), f(S, S, 16, -32, 32, 0.25)
    q, k, v = f(S, D, 21, -8, 8, 0.125), f(S, DKV, 22, -8, 8, 0.125), f(S, DKV, 23, -16, 16, 0.125)
    ta, tc = refs.llm_tokens(S, "prefix"), refs.llm_tokens(S, "causal")
    X, Bm, G, TAB, SC = to_dev(x), to_dev(b), to_dev(g), to_dev(tab), to_dev(sc)
    Q, K, V = to_dev(q), to_dev(k), to_dev(v)
    TA, TC = _tok(ta), _tok(tc)
    out = {t: _zeros(S, D) for t in ("RMS", "ROPE", "SILU", "O", "OU")}
    out.update({t: _zeros(S, S) for t in ("SMA", "SMC")})
    lib.sh_rmsnorm(A(out["RMS"]), A(X), A(G), S, D, D, 1e-5, ALL)
    lib.sh_rope(A(out["ROPE"]), A(X), A(TAB), S, D, D, DH, DH, ALL)
    lib.sh_silu_mul(A(out["SILU"]), A(X), A(Bm), S, D, D, ALL)
    lib.sh_softmax_masked(A(out["SMA"]), A(SC), S, S, S, 0.5, A(TA), A(TA), ALL)
    lib.sh_softmax_masked(A(out["SMC"]), A(SC), S, S, S, 0.5, A(TC), A(TC), ALL)
    assert lib.sh_attention_gqa(A(Q), A(K), A(V), A(out["O"]), S, D, H, Hkv, D, DKV, DKV, D, 0.125, A(TA), ALL) == 0, shops.last_error()
    assert lib.sh_attention_gqa(A(Q), A(K), A(V), A(out["OU"]), S, D, H, Hkv, D, DKV, DKV, D, 0.125, 0, ALL) == 0, shops.last_error()
    want = {"RMS": refs.rmsnorm(x, g, 1e-5), "ROPE": refs.rope(x, tab, DH), "SILU": refs.silu_mul(x, b),
            "SMA": refs.softmax_masked(sc, 0.5, ta, ta), "SMC": refs.softmax_masked(sc, 0.5, tc, tc),
            "O": refs.attention_gqa(q, k, v, H, Hkv, ta), "OU": refs.attention_gqa(q, k, v, H, Hkv)}
    for tag, w in want.items():
        bad, err, _ = refs.close(to_np(out[tag]), w)
        assert bad == 0, f"{tag}: {err}"


@pytest.mark.parametrize("cols", [100, 768, 8192])
def test_rmsnorm_and_masked_softmax_widths(lib, gpu, cols):
    """cols % 8 != 0 takes the element-wise layout; 8192 the widest register-resident row."""
    rows = 40
    x, g = data.normal((rows, cols), 51), data.normal((1, cols), 52, 1.0, 0.1)
    Y = _zeros(rows, cols)
    lib.sh_rmsnorm(A(Y), A(to_dev(x)), A(to_dev(g)), rows, cols, cols, 1e-6, ALL)
    assert refs.close(to_np(Y), refs.rmsnorm(x, g, 1e-6))[0] == 0
    s = data.normal((rows, cols), 53, 0.0, 3.0)
    tq = np.array([(i * 7) % 5 for i in range(rows)], np.uint32)
    tq[3] = refs.LLM_PAD
    tk = np.array([(j * 3) % 6 for j in range(cols)], np.uint32)
    tk[0] = 7                                                   # query classes 0..4 never see key 0
    P = _zeros(rows, cols)
    lib.sh_softmax_masked(A(P), A(to_dev(s)), rows, cols, cols, 0.3, A(_tok(tq)), A(_tok(tk)), ALL)
    bad, err, _ = refs.close(to_np(P), refs.softmax_masked(s, 0.3, tq, tk))
    assert bad == 0, err


@pytest.mark.parametrize("S,dh,H,Hkv", [(64, 64, 4, 2), (100, 128, 2, 1), (36, 36, 3, 1), (256, 64, 6, 6)])
def test_gqa_shapes_masks_and_paths(lib, gpu, S, dh, H, Hkv):
    """Ragged S through the flash kernel, dh = 36 through the per-query kernel, Hkv = H (plain multi-head), and
    four masks: none, causal, all-zero (bidirectional) and a mix with padding rows and unreachable keys."""
    D, DKV = H * dh, Hkv * dh
    q, k, v = data.normal((S, D), 61), data.normal((S, DKV), 62), data.normal((S, DKV), 63)
    Q, K, V = to_dev(q), to_dev(k), to_dev(v)
    mix = np.array([(j % 3) if j % 11 else refs.LLM_PAD for j in range(S)], np.uint32)
    for tok in (None, refs.llm_tokens(S, "causal"), np.zeros(S, np.uint32), mix):
        O = _zeros(S, D)
        T = _tok(tok) if tok is not None else None
        rc = lib.sh_attention_gqa(A(Q), A(K), A(V), A(O), S, D, H, Hkv, D, DKV, DKV, D, 0.125, A(T) if T is not None else 0, ALL)
        assert rc == 0, shops.last_error()
        bad, err, _ = refs.close(to_np(O), refs.attention_gqa(q, k, v, H, Hkv, tok))
        assert bad == 0, err
    O = _zeros(S, dh)                                         # one head through sh_attention_head_masked
    tc = refs.llm_tokens(S, "causal")
    assert lib.sh_attention_head_masked(A(Q), A(K), A(V), A(O), S, dh, D, DKV, DKV, dh, 0.125, A(_tok(tc)), ALL) == 0
    bad, err, _ = refs.close(to_np(O), refs.attention_gqa(q[:, :dh], k[:, :dh], v[:, :dh], 1, 1, tc))
    assert bad == 0, err


def test_rope_heads_in_place_and_silu(lib, gpu):
    rows, dh, nh = 70, 16, 5
    cols = dh * nh
    x = data.normal((rows, cols), 71)
    th = np.outer(np.arange(rows), 1.0 / 10000 ** (np.arange(dh // 2) / (dh // 2)))
    tab = np.concatenate([np.cos(th), np.sin(th)], 1).astype(np.float16)
    X = to_dev(x)
    lib.sh_rope(A(X), A(X), A(to_dev(tab)), rows, cols, cols, dh, dh, ALL)      # in place
    assert refs.close(to_np(X), refs.rope(x, tab, dh))[0] == 0
    a, b = data.normal((rows, 36), 72, 0.0, 4.0), data.normal((rows, 36), 73)
    Y = _zeros(rows, 36)
    lib.sh_silu_mul(A(Y), A(to_dev(a)), A(to_dev(b)), rows, 36, 36, ALL)       # cols % 8 != 0
    assert refs.close(to_np(Y), refs.silu_mul(a, b))[0] == 0


@pytest.mark.parametrize("grid,D,s", [(8, 64, 2), (6, 12, 3), (26, 768, 13)])
def test_pixel_shuffle_bit_exact(lib, gpu, grid, D, s):
    """Every 16-bit pattern (NaN payloads included) moves unchanged; D = 12 takes the element-wise kernel."""
    src = np.random.default_rng(81).integers(0, 1 << 16, (grid * grid, D)).astype(np.uint16).view(np.float16)
    g = grid // s
    Dst = _zeros(g * g, D * s * s)
    lib.sh_pixel_shuffle(A(Dst), A(to_dev(src)), grid, D, s, ALL)
    assert np.array_equal(to_np(Dst).view(np.uint16), refs.pixel_shuffle(src.view(np.uint16), grid, s))


def test_llm_argument_errors(lib, gpu):
    one = 1 << 20
    assert lib.sh_attention_gqa(one, one, one, one, 256, 960, 15, 4, 960, 256, 256, 960, 0.125, 0, ALL) == -1   # H % Hkv
    assert lib.sh_attention_gqa(one, one, one, one, 512, 960, 15, 5, 960, 320, 320, 960, 0.125, 0, ALL) == -1   # S > 256
    assert lib.sh_attention_head_masked(one, one, one, one, 64, 64, 64, 64, 64, 64, -0.1, 0, ALL) == -1        # scale <= 0
    lib.sh_rmsnorm(one, one, one, 4, 30, 30, 1e-6, ALL)                                                       # cols % 4
    assert shops.last_error()[0] == -1
    lib.sh_rope(one, one, one, 4, 60, 60, 12, 12, ALL)                                                       # dh % 8
    assert shops.last_error()[0] == -1
    lib.sh_softmax_masked(one, one, 4, 64, 64, 0.0, one, one, ALL)                                           # scale <= 0
    assert shops.last_error()[0] == -1
