"""sh_gemm_ex_wt (the weight given as W^T, [N, K]) against sh_gemm_ex on the same operands: every W^T tile
configuration accumulates K in the order of the direct-to-LDS kernels, and the register-staged W^T fallback in the
order of the register-staged kernels, so the stores are bit-identical; epilogues, split-K, partial tiles, strided
and unaligned views, and the encoder's shapes; plus the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import K2_CFGS, REGSTAGED_CFGS, WT_CFGS, codes, to_dev, to_np
from oracle import refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
A = shops.addr
FALLBACK_CFGS = REGSTAGED_CFGS   # register-staged tiles (both layouts)


def _wt(w):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(w.T)).cuda()
    from conftest import _KEEP
    _KEEP.append(t)
    return t


@pytest.mark.parametrize("cfg_index", list(WT_CFGS) + list(FALLBACK_CFGS))
def test_wt_config_matches_natural_layout_bitwise(lib, gpu, cfg_index, monkeypatch):
    import torch
    M, N, K = 328, 200, 192                       # partial tiles in M and N, K % 64 == 0
    x = data.normal((M, K), 31)
    w = data.normal((K, N), 32, std=1 / np.sqrt(K))
    X, W, WT = to_dev(x), to_dev(w), _wt(w)
    ref_cfg = cfg_index if cfg_index in FALLBACK_CFGS else K2_CFGS[0]
    monkeypatch.setenv("SH_GEMM_CFG", str(ref_cfg))
    if cfg_index in FALLBACK_CFGS:
        K = 136                                   # K % 64 != 0: W^T calls take the register-staged tiles
        x, w = x[:, :K], w[:K]
        X, W, WT = to_dev(x), to_dev(w), _wt(w)
    Zr = torch.full((M + 3, 208), 7.0, dtype=torch.float16, device="cuda")
    assert lib.sh_gemm_ex(A(X), A(W), A(Zr), M, N, K, K, N, 208, None, None) == 0, shops.last_error()
    monkeypatch.setenv("SH_GEMM_CFG", str(cfg_index))
    Z = torch.full((M + 3, 208), 7.0, dtype=torch.float16, device="cuda")
    assert lib.sh_gemm_ex_wt(A(X), A(WT), A(Z), M, N, K, K, K, 208, None, None) == 0, shops.last_error()
    z = to_np(Z)
    assert np.array_equal(codes(Z), codes(Zr)), cfg_index
    assert (z[:M, N:] == 7.0).all() and (z[M:] == 7.0).all()
    bad, err, _ = refs.close(z[:M, :N], refs.gemm(x, w))
    assert bad == 0, err


@pytest.mark.parametrize("epi", ["bias16", "bias32_gelu", "residual", "accumulate", "split3"])
def test_wt_epilogues_match_natural_layout_bitwise(lib, gpu, epi):
    import torch
    M, N, K = 520, 392, 448
    x = data.normal((M, K), 41)
    w = data.normal((K, N), 42, std=1 / np.sqrt(K))
    b16 = data.normal((1, N), 43, std=0.3).astype(np.float16)
    b32 = data.normal((1, N), 44, std=0.3).astype(np.float32)
    r = data.normal((M, N), 45)
    X, W, WT, B16, R = to_dev(x), to_dev(w), _wt(w), to_dev(b16), to_dev(r)
    B32 = torch.from_numpy(b32).cuda()
    cfg = shops.cfg(accumulate=1) if epi == "accumulate" else None
    e = {"bias16": shops.epi(bias=A(B16)),
         "bias32_gelu": shops.epi(bias=A(B32), bias_fmt=shops.SH_BIAS_FP32, act=shops.SH_ACT_GELU),
         "residual": shops.epi(bias=A(B16), residual=A(R), ldr=N),
         "accumulate": shops.epi(),
         "split3": shops.epi(bias=A(B16), splits=3)}[epi]
    z0 = data.normal((M, N), 46)
    Zr, Z = to_dev(z0), to_dev(z0)
    assert lib.sh_gemm_ex(A(X), A(W), A(Zr), M, N, K, K, N, N, cfg, e) == 0, shops.last_error()
    assert lib.sh_gemm_ex_wt(A(X), A(WT), A(Z), M, N, K, K, K, N, cfg, e) == 0, shops.last_error()
    assert np.array_equal(codes(Z), codes(Zr)), epi


def test_wt_unaligned_and_strided_views(lib, gpu):
    """Odd N and K with operands one element into their buffers (register-staged W^T path), and a W^T view with
    ldwt > K (a column block of a wider matrix)."""
    import torch
    M, N, K = 70, 45, 37
    x = data.normal((M, K + 1), 51)
    wtb = data.normal((N + 3, K + 5), 52, std=0.2)             # W^T buffer; the view starts one element in
    X, WTb = to_dev(x), to_dev(wtb)
    Z = torch.zeros((M, N + 2), dtype=torch.float16, device="cuda")
    rc = lib.sh_gemm_ex_wt(A(X, 1), A(WTb, 1), A(Z, 1), M, N, K, K + 1, K + 5, N + 2, None, None)
    assert rc == 0, shops.last_error()
    want = refs.gemm(x[:, 1:], np.ascontiguousarray(wtb[:N, 1:K + 1].T))
    bad, err, _ = refs.close(to_np(Z)[:, 1:N + 1], want)
    assert bad == 0, err
    assert lib.sh_gemm_ex_wt(A(X), A(WTb), A(Z), M, N, K, K + 1, K - 1, N + 2, None, None) == -1     # ldwt < K


@pytest.mark.parametrize("N,K,epi", [(2304, 768, "bias"), (768, 768, "res"), (3072, 768, "gelu"), (768, 3072, "res")])
def test_wt_encoder_shapes_match_natural_layout(lib, gpu, N, K, epi):
    """The encoder's four GEMM shapes (M = 8192) with their epilogues: W^T and W layouts store the same bits,
    within tolerance of the oracle (checked on a sample of rows)."""
    import torch
    M = 8192
    x = data.normal((M, K), 61)
    w = data.normal((K, N), 62, std=0.02)
    b = data.normal((1, N), 63, std=0.02).astype(np.float16)
    r = data.normal((M, N), 64)
    X, W, WT, Bb, R = to_dev(x), to_dev(w), _wt(w), to_dev(b), to_dev(r)
    e = {"bias": shops.epi(bias=A(Bb)), "gelu": shops.epi(bias=A(Bb), act=shops.SH_ACT_GELU),
         "res": shops.epi(bias=A(Bb), residual=A(R), ldr=N)}[epi]
    Zr = torch.empty((M, N), dtype=torch.float16, device="cuda")
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    assert lib.sh_gemm_ex(A(X), A(W), A(Zr), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    assert lib.sh_gemm_ex_wt(A(X), A(WT), A(Z), M, N, K, K, K, N, None, e) == 0, shops.last_error()
    assert np.array_equal(codes(Z), codes(Zr))
    rows = np.arange(0, M, 61)
    want = refs.r16(refs.r16(refs.gemm(x[rows], w)) + b.astype(np.float32))
    if epi == "gelu":
        want = refs.gelu(want)
    if epi == "res":
        want = want + r[rows].astype(np.float32)
    bad, err, _ = refs.close(to_np(Z)[rows], want)
    assert bad == 0, err
