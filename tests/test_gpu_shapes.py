"""Seeded random shapes through the path's entry points, each against the oracle. The fixed-shape tests pin the
BASELINE configs, every tile configuration and each epilogue on chosen sizes; these draw sizes, leading dimensions,
buffer offsets (16-byte aligned or not), epilogues, split counts and attention geometries at random, so that
combinations the fixed cases do not name still meet the oracle. Each case's parameters come from its own seed
(1000 + case): a failure names a reproducible case."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import _KEEP, codes, to_dev, to_np
from oracle import refs
from softhier_mlir_amd import shops

pytestmark = pytest.mark.gpu
A = shops.addr
ALL = shops.SH_ALL


def _rng(case: int) -> np.random.Generator:
    return np.random.default_rng(1000 + case)


def _fp16(r: np.random.Generator, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    return r.uniform(lo, hi, size=shape).astype(np.float16)


def _buf(r: np.random.Generator, rows: int, cols: int, ld: int, off: int) -> np.ndarray:
    """A [rows, cols] operand inside a padded fp16 buffer: row stride ld, starting `off` elements in."""
    flat = _fp16(r, off + rows * ld + 8)
    return flat


def _view(flat: np.ndarray, rows: int, cols: int, ld: int, off: int) -> np.ndarray:
    return flat[off:off + rows * ld].reshape(rows, ld)[:, :cols]


@pytest.mark.parametrize("case", range(48))
def test_random_gemm(lib, gpu, case):
    """sh_gemm_ex on M, N, K from 1 up, padded leading dimensions, offsets that break 16-byte alignment, each
    epilogue (fp16 / fp32 bias, GELU, residual, accumulate) and 1-3 K ranges."""
    import torch
    r = _rng(case)
    M, N, K = int(r.integers(1, 600)), int(r.integers(1, 700)), int(r.integers(1, 900))
    ldx, ldw, ldz = (n + int(r.choice([0, 0, 8, 3])) for n in (K, N, N))
    ox, ow, oz = (int(r.choice([0, 0, 1])) for _ in range(3))
    kind = str(r.choice(["none", "bias16", "bias32", "gelu", "res", "acc"]))
    splits = int(r.choice([1, 1, 2, 3]))
    fx, fw = _buf(r, M, K, ldx, ox), _buf(r, K, N, ldw, ow)
    fw = (fw.astype(np.float32) / np.float32(np.sqrt(K))).astype(np.float16)
    fz = _buf(r, M, N, ldz, oz)
    x, w, z0 = _view(fx, M, K, ldx, ox), _view(fw, K, N, ldw, ow), _view(fz, M, N, ldz, oz)
    X, W, Z = to_dev(fx), to_dev(fw), to_dev(fz)
    want = refs.gemm(x, w)
    cfg, e = None, shops.epi(splits=splits)
    if kind in ("bias16", "gelu"):
        b = _fp16(r, (1, N), -0.1, 0.1)
        B_ = to_dev(b)
        e = shops.epi(bias=A(B_), act=shops.SH_ACT_GELU if kind == "gelu" else shops.SH_ACT_NONE, splits=splits)
        want = refs.r16(refs.r16(want) + b.astype(np.float32))
        if kind == "gelu":
            want = refs.gelu(want)
    elif kind == "bias32":
        b32 = r.uniform(-0.1, 0.1, size=(1, N)).astype(np.float32)
        B_ = torch.from_numpy(b32).cuda()
        e = shops.epi(bias=A(B_), bias_fmt=shops.SH_BIAS_FP32, splits=splits)
        want = refs.r16(refs.r16(want) + b32)
    elif kind == "res":
        ldr = N + int(r.choice([0, 8]))
        fr = _buf(r, M, N, ldr, 0)
        R_ = to_dev(fr)
        e = shops.epi(residual=A(R_), ldr=ldr, splits=splits)
        want = refs.r16(refs.r16(want) + _view(fr, M, N, ldr, 0).astype(np.float32))
    elif kind == "acc":
        cfg = shops.cfg(accumulate=1)
        want = refs.r16(z0.astype(np.float32) + refs.r16(want))
    rc = lib.sh_gemm_ex(A(X, ox), A(W, ow), A(Z, oz), M, N, K, ldx, ldw, ldz, cfg, e)
    assert rc == 0, (case, M, N, K, kind, splits, shops.last_error())
    got = _view(to_np(Z), M, N, ldz, oz)
    bad, err, _ = refs.close(got, want)
    assert bad == 0, (case, M, N, K, ldx, ldw, ldz, ox, ow, oz, kind, splits, err)
    # the padding between rows and past the operand is untouched
    untouched = np.ones(fz.shape, bool)
    _view(untouched, M, N, ldz, oz)[:] = False
    assert np.array_equal(codes(Z)[untouched], fz.view(np.uint16)[untouched]), (case, "wrote outside the output view")


ROW_OPS = ("layernorm", "layernorm_ld", "softmax", "gelu", "add", "add_bias", "scale", "transpose")


@pytest.mark.parametrize("case", range(40))
def test_random_rowops(lib, gpu, case):
    """The row ops on widths from 1 to 9000 (the register-resident, wide and scalar paths), padded views and
    offsets that break 16-byte alignment; transpose bit for bit."""
    import torch
    r = _rng(100 + case)
    op = ROW_OPS[case % len(ROW_OPS)]
    rows, cols = int(r.integers(1, 1500)), int(r.choice([int(r.integers(1, 300)), int(r.integers(300, 4200)),
                                                         int(r.integers(4200, 9000))]))
    ld = cols + int(r.choice([0, 0, 8, 5]))
    off = int(r.choice([0, 0, 3]))
    fx = _buf(r, rows, cols, ld, off)
    if op == "softmax":
        fx = (fx.astype(np.float32) * 4).astype(np.float16)
    x = _view(fx, rows, cols, ld, off)
    X = to_dev(fx)
    if op == "transpose":
        ldt = rows + int(r.choice([0, 8, 1]))
        T = torch.full((cols * ldt + 8,), 3.0, dtype=torch.float16, device="cuda")
        lib.sh_transpose(A(T), A(X, off), rows, cols, ld, ldt, ALL)
        got = codes(T)[:cols * ldt].reshape(cols, ldt)[:, :rows]
        assert np.array_equal(got, refs.transpose(x.view(np.uint16))), (case, rows, cols, ld, ldt, off)
        return
    fy = np.full(off + rows * ld + 8, 7.0, np.float16)
    Y = to_dev(fy)
    g, b = _fp16(r, (1, cols), 0.5, 1.5), _fp16(r, (1, cols), -0.5, 0.5)
    G, Bb = to_dev(g), to_dev(b)
    if op == "layernorm":
        lib.sh_layernorm(A(Y, off), A(X, off), A(G), A(Bb), rows, cols, ld, 1e-5, ALL)
        want = refs.layernorm(x, g, b, 1e-5)
    elif op == "layernorm_ld":
        ldy = cols + 8
        fy = np.full(rows * ldy + 8, 7.0, np.float16)
        Y = to_dev(fy)
        lib.sh_layernorm_ld(A(Y), A(X, off), A(G), A(Bb), rows, cols, ldy, ld, 1e-6)
        got = to_np(Y)[:rows * ldy].reshape(rows, ldy)[:, :cols]
        bad, err, _ = refs.close(got, refs.layernorm(x, g, b, 1e-6))
        assert bad == 0, (case, op, rows, cols, ld, off, err)
        return
    elif op == "softmax":
        s = float(r.choice([0.125, 0.5, -0.25]))
        lib.sh_softmax_rows(A(Y, off), A(X, off), rows, cols, ld, s, ALL)
        want = refs.softmax(x, s)
    elif op == "gelu":
        lib.sh_gelu(A(Y, off), A(X, off), rows, cols, ld, ALL)
        want = refs.gelu(x)
    elif op == "add":
        fb = _buf(r, rows, cols, ld, off)
        Bt = to_dev(fb)
        lib.sh_add(A(Y, off), A(X, off), A(Bt, off), rows, cols, ld, ALL)
        want = refs.add(x, _view(fb, rows, cols, ld, off))
    elif op == "add_bias":
        lib.sh_add_bias(A(Y, off), A(X, off), A(Bb), rows, cols, ld, ALL)
        want = refs.add_bias(x, b)
    else:
        s = float(r.uniform(-2, 2))
        lib.sh_scale(A(Y, off), A(X, off), rows, cols, ld, s, ALL)
        want = refs.scale(x, s)
    got = _view(to_np(Y), rows, cols, ld, off)
    bad, err, _ = refs.close(got, want)
    assert bad == 0, (case, op, rows, cols, ld, off, err)
    untouched = np.ones(fy.shape, bool)
    _view(untouched, rows, cols, ld, off)[:] = False
    assert np.array_equal(codes(Y)[untouched], fy.view(np.uint16)[untouched]), (case, op, "wrote outside the view")


@pytest.mark.parametrize("case", range(24))
def test_random_attention(lib, gpu, case):
    """sh_attention_batched with S from 4 up (ragged key blocks and partial query blocks), head widths 32 / 64 /
    80 / 128, 1-4 heads, 1-3 sequences, packed or separate operands and scales on either side of the fold limit."""
    import torch
    r = _rng(200 + case)
    B, H = int(r.integers(1, 4)), int(r.integers(1, 5))
    dh = int(r.choice([32, 64, 64, 80, 128]))
    S = 4 * int(r.integers(1, 80))
    D = H * dh
    scale = float(r.choice([1.0 / np.sqrt(dh), 0.05, 0.9]))
    packed = bool(r.integers(0, 2))
    if packed:
        qkv = _fp16(r, (B * S, 3 * D))
        q, k, v, ld = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], 3 * D
        T = to_dev(qkv)
        pq, pk, pv = A(T), A(T, D), A(T, 2 * D)
    else:
        q, k, v = (_fp16(r, (B * S, D)) for _ in range(3))
        ld = D
        Q, K_, V = to_dev(q), to_dev(k), to_dev(v)
        pq, pk, pv = A(Q), A(K_), A(V)
    O = torch.full((B * S, D), 7.0, dtype=torch.float16, device="cuda")
    rc = lib.sh_attention_batched(pq, pk, pv, A(O), B, S, D, H, ld, ld, ld, D, S * ld, S * ld, S * ld, S * D, scale, 0)
    assert rc == 0, (case, B, S, H, dh, shops.last_error())
    want = refs.attention_batched(q, k, v, B, H, scale)
    bad, err, _ = refs.close(to_np(O), want)
    assert bad == 0, (case, B, S, H, dh, scale, packed, err)


@pytest.mark.parametrize("case", range(16))
def test_random_gemm_wt(lib, gpu, case):
    """sh_gemm_ex_wt (the weight given as W^T, [N, ldwt]) on random shapes, views and epilogues, against the oracle."""
    import torch
    r = _rng(300 + case)
    M, N, K = int(r.integers(1, 600)), int(r.integers(1, 700)), int(r.integers(1, 900))
    ldx, ldwt, ldz = (n + int(r.choice([0, 0, 8, 3])) for n in (K, K, N))
    ox, ow = (int(r.choice([0, 0, 1])) for _ in range(2))
    kind = str(r.choice(["none", "bias16", "gelu", "res"]))
    splits = int(r.choice([1, 1, 2, 3]))
    fx, fwt = _buf(r, M, K, ldx, ox), _buf(r, N, K, ldwt, ow)
    fwt = (fwt.astype(np.float32) / np.float32(np.sqrt(K))).astype(np.float16)
    x, wt = _view(fx, M, K, ldx, ox), _view(fwt, N, K, ldwt, ow)
    X, WT = to_dev(fx), to_dev(fwt)
    Z = torch.full((M * ldz + 8,), 7.0, dtype=torch.float16, device="cuda")
    want = refs.gemm(x, wt.T)
    e = shops.epi(splits=splits)
    if kind in ("bias16", "gelu"):
        b = _fp16(r, (1, N), -0.1, 0.1)
        B_ = to_dev(b)
        e = shops.epi(bias=A(B_), act=shops.SH_ACT_GELU if kind == "gelu" else shops.SH_ACT_NONE, splits=splits)
        want = refs.r16(refs.r16(want) + b.astype(np.float32))
        if kind == "gelu":
            want = refs.gelu(want)
    elif kind == "res":
        fr = _buf(r, M, N, N, 0)
        R_ = to_dev(fr)
        e = shops.epi(residual=A(R_), ldr=N, splits=splits)
        want = refs.r16(refs.r16(want) + _view(fr, M, N, N, 0).astype(np.float32))
    rc = lib.sh_gemm_ex_wt(A(X, ox), A(WT, ow), A(Z), M, N, K, ldx, ldwt, ldz, None, e)
    assert rc == 0, (case, M, N, K, kind, splits, shops.last_error())
    got = to_np(Z)[:M * ldz].reshape(M, ldz)[:, :N]
    bad, err, _ = refs.close(got, want)
    assert bad == 0, (case, M, N, K, ldx, ldwt, ldz, ox, ow, kind, splits, err)


def _f32(shape):
    import torch
    t = torch.empty(shape, dtype=torch.float32, device="cuda")
    _KEEP.append(t)
    return t


@pytest.mark.parametrize("case", range(16))
def test_random_layernorm_fold(lib, gpu, case):
    """A producer GEMM writing row partials (N = 32 k) handing its rows to a GEMM that folds their LayerNorm (from
    those partials, or from sh_row_stats), with or without GELU: against LayerNorm -> GEMM -> bias [-> GELU] on the
    producer's stored rows."""
    import torch
    r = _rng(400 + case)
    M, K, N = int(r.integers(1, 700)), 32 * int(r.integers(1, 33)), int(r.integers(1, 700))
    K0 = 8 * int(r.integers(1, 38))              # (row partials need 16-byte aligned rows)
    act = int(r.integers(0, 2))
    from_partials = bool(r.integers(0, 2))
    eps = 1e-6
    x0, w0 = _fp16(r, (M, K0)), (_fp16(r, (K0, K)).astype(np.float32) * np.float32(2 / np.sqrt(K0))).astype(np.float16)
    w = (_fp16(r, (K, N)).astype(np.float32) / np.float32(np.sqrt(K))).astype(np.float16)
    g, be, b = _fp16(r, (1, K), 0.5, 1.5), _fp16(r, (1, K), -0.3, 0.3), _fp16(r, (1, N), -0.3, 0.3)
    X0, W0, W, G, BE, Bb = (to_dev(a) for a in (x0, w0, w, g, be, b))
    X = torch.empty((M, K), dtype=torch.float16, device="cuda")
    P = _f32((M, K // 32, 2))
    e0 = shops.epi(stats_out=A(P)) if from_partials else None
    assert lib.sh_gemm_ex(A(X0), A(W0), A(X), M, K, K0, K0, K, K, None, e0) == 0, (case, shops.last_error())
    WP = torch.empty((K, N), dtype=torch.float16, device="cuda")
    C, D = _f32((N + 4,)), _f32((N + 4,))
    lib.sh_ln_fold(A(WP), A(C), A(D), A(W), A(G), A(BE), A(Bb), K, N, N, N)
    if from_partials:
        e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(P), ln_c=A(C), ln_parts=K // 32,
                      ln_eps=eps)
    else:
        S = _f32((M, 2))
        lib.sh_row_stats(A(S), A(X), M, K, K, eps)
        e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(S), ln_c=A(C))
    assert shops.last_error()[0] == 0, (case, shops.last_error())
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    assert lib.sh_gemm_ex(A(X), A(WP), A(Z), M, N, K, K, N, N, None, e) == 0, (case, shops.last_error())
    x = to_np(X)                                          # the producer's stored rows (its own tests pin them)
    want = refs.r16(refs.add_bias(refs.r16(refs.gemm(refs.r16(refs.layernorm(x, g, be, eps)), w)), b))
    if act:
        want = refs.gelu(want)
    bad, err, _ = refs.close(to_np(Z), want)
    assert bad == 0, (case, M, K, N, K0, act, from_partials, err)
