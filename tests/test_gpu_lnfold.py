"""LayerNorm folded into the next GEMM: sh_row_stats (per-row mean and 1 / sqrt(var + eps)), sh_ln_fold (W' =
r16(gamma W), c = 1^T W', d = beta^T W + b) and sh_gemm_ex with sh_gemm_epi.ln_stats / ln_c, which stores
LN(x) . W + b (then GELU / residual) in one pass over x.

The statistics are pinned by float64 mean / variance; W' bit-exactly by its definition; the folded GEMM against the
oracle's unfused sequence (layernorm -> r16 -> gemm -> bias -> r16 -> GELU, siglip_ref.py:24-40), within the
encoder's fp16 tolerance (2e-2 absolute + 1e-2 relative), since the fold rounds gamma W where the reference rounds
LN(x). Tile configurations that apply the fold on their fp32 accumulators store identical bits, and the fp32
partials path (one K range, reduced) stores those bits too."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import K2_CFGS, K5_CFGS, codes, to_dev, to_np
from oracle import refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
A = shops.addr
REG_CFGS = list(K5_CFGS)      # W layout tiles with the fold in registers
EPS = 1e-6


def _f32_dev(a):
    import torch
    from conftest import _KEEP
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
    _KEEP.append(t)
    return t


def _empty32(*shape):
    import torch
    from conftest import _KEEP
    t = torch.empty(shape, dtype=torch.float32, device="cuda")
    _KEEP.append(t)
    return t


def _stats_f64(x):
    x = np.asarray(x, np.float64)
    mu = x.mean(1)
    return mu, 1.0 / np.sqrt(x.var(1) + EPS)


@pytest.mark.parametrize("rows,cols,ld", [(8192, 768, 768), (37, 768, 776), (300, 256, 256), (129, 1024, 1024),
                                          (64, 3072, 3072), (65, 4096, 4104), (1, 8, 8)])
def test_row_stats_match_float64(lib, gpu, rows, cols, ld):
    x = data.normal((rows, ld), 11 + cols, mean=0.5, std=2.0)
    x[0] = 1.25                                   # variance 0: r = 1 / sqrt(eps)
    X = to_dev(x)
    S = _empty32(rows + 1, 2)
    S[rows] = 1234.5
    lib.sh_row_stats(A(S), A(X), rows, cols, ld, EPS)
    assert shops.last_error()[0] == 0, shops.last_error()
    s = to_np(S)
    mu, r = _stats_f64(refs.f32(x)[:, :cols])
    assert np.allclose(s[:rows, 0], mu, rtol=0, atol=1e-5 * np.abs(refs.f32(x)).max())
    assert np.allclose(s[:rows, 1], r, rtol=1e-5, atol=0)
    assert abs(s[0, 1] - 1e3) <= 1e-2
    assert (s[rows] == 1234.5).all()


def test_row_stats_argument_errors(lib, gpu):
    X = to_dev(data.normal((4, 768), 1))
    S = _empty32(4, 2)
    lib.sh_row_stats(A(S), A(X), 4, 761, 768, EPS)            # cols % 8 != 0
    assert shops.last_error()[0] == -1
    lib.sh_row_stats(A(S) + 4, A(X), 4, 768, 768, EPS)        # stats not 8-byte aligned
    assert shops.last_error()[0] == -1


@pytest.mark.parametrize("K,N,ldw,ldwp,bias", [(768, 2304, 2304, 2304, True), (768, 3072, 3080, 3072, False),
                                                (100, 37, 40, 48, True)])
def test_ln_fold_weights(lib, gpu, K, N, ldw, ldwp, bias):
    import torch
    w = data.normal((K, ldw), 21, std=1 / np.sqrt(K))
    g = (1.0 + data.normal((1, K), 22, std=0.2)).astype(np.float16)
    be = data.normal((1, K), 23, std=0.2).astype(np.float16)
    b = data.normal((1, N), 24, std=0.2).astype(np.float16)
    W, G, BE, Bb = to_dev(w), to_dev(g), to_dev(be), to_dev(b)
    WP = torch.full((K, ldwp), 7.0, dtype=torch.float16, device="cuda")
    C, D = _empty32(N), _empty32(N)
    lib.sh_ln_fold(A(WP), A(C), A(D), A(W), A(G), A(BE), A(Bb) if bias else 0, K, N, ldw, ldwp)
    assert shops.last_error()[0] == 0, shops.last_error()
    wf = refs.f32(w)[:, :N]
    wp = (refs.f32(g).reshape(-1, 1) * wf).astype(np.float16)            # fp32 product, one rounding
    assert np.array_equal(codes(WP)[:, :N], wp.view(np.uint16))
    assert (to_np(WP)[:, N:] == 7.0).all()
    # fp32 sums of K terms: |error| <= K u sum |term| (u = 2^-24 per rounding, doubled for the products)
    c = wp.astype(np.float64).sum(0)
    bw = refs.f32(be).astype(np.float64).reshape(-1, 1) * wf
    d = bw.sum(0) + (refs.f32(b)[0] if bias else 0.0)
    u = 2.0 ** -24
    assert np.all(np.abs(to_np(C) - c) <= K * u * np.abs(wp.astype(np.float64)).sum(0))
    assert np.all(np.abs(to_np(D) - d) <= 2 * (K + 1) * u * (np.abs(bw).sum(0) + np.abs(d)))


def _problem(M, N, K, seed, mean=0.3):
    x = (data.normal((M, K), seed, std=1.5) + mean).astype(np.float16)
    w = data.normal((K, N), seed + 1, std=1 / np.sqrt(K))
    g = (1.0 + data.normal((1, K), seed + 2, std=0.2)).astype(np.float16)
    be = data.normal((1, K), seed + 3, std=0.2).astype(np.float16)
    b = data.normal((1, N), seed + 4, std=0.2).astype(np.float16)
    return x, w, g, be, b


def _fold(lib, X, W, G, BE, Bb, M, N, K):
    import torch
    from conftest import _KEEP
    WP = torch.empty((K, N), dtype=torch.float16, device="cuda")
    _KEEP.append(WP)
    C, D, S = _empty32(N + 4), _empty32(N + 4), _empty32(M, 2)
    lib.sh_ln_fold(A(WP), A(C), A(D), A(W), A(G), A(BE), A(Bb), K, N, N, N)
    lib.sh_row_stats(A(S), A(X), M, K, K, EPS)
    assert shops.last_error()[0] == 0, shops.last_error()
    return WP, C, D, S


def _want(x, w, g, be, b, act, res=None):
    ln = refs.r16(refs.layernorm(x, g, be, EPS))
    z = refs.r16(refs.add_bias(refs.r16(refs.gemm(ln, w)), b))
    if act:
        z = refs.r16(refs.gelu(z))
    if res is not None:
        z = refs.r16(refs.add(z, res))
    return z


@pytest.mark.parametrize("M,N,K,act", [(8192, 2304, 768, 0), (8192, 3072, 768, 1), (520, 768, 768, 0),
                                       (328, 192, 192, 1)])
def test_folded_gemm_matches_unfused_layernorm_gemm(lib, gpu, M, N, K, act):
    import torch
    x, w, g, be, b = _problem(M, N, K, 50 + N)
    X, W, G, BE, Bb = to_dev(x), to_dev(w), to_dev(g), to_dev(be), to_dev(b)
    WP, C, D, S = _fold(lib, X, W, G, BE, Bb, M, N, K)
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(S), ln_c=A(C))
    assert lib.sh_gemm_ex(A(X), A(WP), A(Z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    bad, err, _ = refs.close(to_np(Z), _want(x, w, g, be, b, act))
    assert bad == 0, err


def test_folded_gemm_with_residual(lib, gpu):
    import torch
    M, N, K = 512, 768, 768
    x, w, g, be, b = _problem(M, N, K, 70)
    r = data.normal((M, N), 75)
    X, W, G, BE, Bb, R = to_dev(x), to_dev(w), to_dev(g), to_dev(be), to_dev(b), to_dev(r)
    WP, C, D, S = _fold(lib, X, W, G, BE, Bb, M, N, K)
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, residual=A(R), ldr=N, ln_stats=A(S), ln_c=A(C))
    assert lib.sh_gemm_ex(A(X), A(WP), A(Z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    bad, err, _ = refs.close(to_np(Z), _want(x, w, g, be, b, 0, res=r))
    assert bad == 0, err


@pytest.mark.parametrize("act", [0, 1])
def test_fold_configs_and_partials_path_store_identical_bits(lib, gpu, act, monkeypatch):
    """Every register-epilogue tile, and the fp32 partials path (one K range, reduced; taken when ln_c is not
    16-byte aligned) of a direct-to-LDS tile with or without that epilogue, store the same bits: the accumulators
    are summed over K in one order and the fold is the same fp32 expression."""
    import torch
    M, N, K = 520, 584, 448                     # partial tiles in M and N
    x, w, g, be, b = _problem(M, N, K, 90)
    X, W, G, BE, Bb = to_dev(x), to_dev(w), to_dev(g), to_dev(be), to_dev(b)
    WP, C, D, S = _fold(lib, X, W, G, BE, Bb, M, N, K)
    C1 = _empty32(N + 1)                        # c one element into its buffer: 4-byte, not 16-byte aligned
    C1[1:N + 1] = C[:N]
    runs = {}
    for cfg in REG_CFGS + [f"partials{K2_CFGS[0]}", f"partials{K2_CFGS[3]}", f"partials{K5_CFGS[0]}"]:
        Z = torch.full((M, N), 3.0, dtype=torch.float16, device="cuda")
        if str(cfg).startswith("partials"):
            monkeypatch.setenv("SH_GEMM_CFG", cfg[8:])
            e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(S), ln_c=A(C1, 1))
        else:
            monkeypatch.setenv("SH_GEMM_CFG", str(cfg))
            e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(S), ln_c=A(C))
        assert lib.sh_gemm_ex(A(X), A(WP), A(Z), M, N, K, K, N, N, None, e) == 0, (cfg, shops.last_error())
        runs[cfg] = codes(Z)
    first = runs[REG_CFGS[0]]
    for cfg, z in runs.items():
        assert np.array_equal(z, first), cfg
    bad, err, _ = refs.close(to_np(Z), _want(x, w, g, be, b, act))
    assert bad == 0, err


def test_fold_split_k_within_tolerance(lib, gpu):
    import torch
    M, N, K = 256, 768, 3072
    x, w, g, be, b = _problem(M, N, K, 110)
    X, W, G, BE, Bb = to_dev(x), to_dev(w), to_dev(g), to_dev(be), to_dev(b)
    WP, C, D, S = _fold(lib, X, W, G, BE, Bb, M, N, K)
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, splits=4, ln_stats=A(S), ln_c=A(C))
    assert lib.sh_gemm_ex(A(X), A(WP), A(Z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    bad, err, _ = refs.close(to_np(Z), _want(x, w, g, be, b, 0))
    assert bad == 0, err


def test_fold_argument_errors(lib, gpu):
    import torch
    M, N, K = 256, 256, 256
    X = to_dev(data.normal((M, K), 1))
    W = to_dev(data.normal((K, N), 2))
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    S, C, D = _empty32(M, 2), _empty32(N), _empty32(N)
    B16 = to_dev(np.zeros((1, N), np.float16))
    bad = [shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, ln_stats=A(S)),                 # no c
           shops.epi(bias=A(B16), ln_stats=A(S), ln_c=A(C)),                                 # fp16 bias
           shops.epi(ln_stats=A(S), ln_c=A(C))]                                              # no d
    for e in bad:
        assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, e) == -1
    e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, ln_stats=A(S), ln_c=A(C))
    assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, shops.cfg(accumulate=1), e) == -1


# ---- row partials written by the producing GEMM (sh_gemm_epi.stats_out) and combined by the consumer ----------
def _partials_f64(z):
    """(sum, M2) of every 32 columns of each row, float64."""
    z = np.asarray(z, np.float64)
    M, N = z.shape
    b = z.reshape(M, N // 32, 32)
    s = b.sum(2)
    return s, ((b - s[..., None] / 32) ** 2).sum(2)


def _producer(M, N, K, seed):
    a = data.normal((M, K), seed)
    w = data.normal((K, N), seed + 1, std=1 / np.sqrt(K))
    b = data.normal((1, N), seed + 2, std=0.3)
    r = (data.normal((M, N), seed + 3, std=2.0) + 0.7).astype(np.float16)
    return a, w, b, r


def test_row_partials_match_float64_and_agree_across_tiles(lib, gpu, monkeypatch):
    """A GEMM with bias + residual that also writes row partials: the pairs match float64 sums over the stored
    fp16 output; every register-epilogue tile writes the same pairs and outputs bit for bit (the same 32 values
    summed in the same order), and the split-K path (the reduction writes them) agrees within fp32 rounding."""
    import torch
    M, N, K = 520, 768, 448
    a, w, b, r = _producer(M, N, K, 130)
    X, W, Bb, R = to_dev(a), to_dev(w), to_dev(b), to_dev(r)
    P = N // 32
    runs = {}
    for cfg in REG_CFGS + ["split3"]:
        Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
        St = _empty32(M, P, 2)
        if cfg == "split3":
            monkeypatch.delenv("SH_GEMM_CFG", raising=False)
            e = shops.epi(bias=A(Bb), residual=A(R), ldr=N, stats_out=A(St), splits=3)
        else:
            monkeypatch.setenv("SH_GEMM_CFG", str(cfg))
            e = shops.epi(bias=A(Bb), residual=A(R), ldr=N, stats_out=A(St))
        assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, e) == 0, (cfg, shops.last_error())
        runs[cfg] = (codes(Z), to_np(St))
    z0, st0 = runs[REG_CFGS[0]]
    for cfg in REG_CFGS:
        assert np.array_equal(runs[cfg][0], z0), cfg
        assert np.array_equal(runs[cfg][1].view(np.uint32), st0.view(np.uint32)), cfg
    s, m2 = _partials_f64(z0.view(np.float16))
    u = 2.0 ** -24
    mag = np.abs(z0.view(np.float16).astype(np.float64)).reshape(M, P, 32).sum(2)
    assert np.all(np.abs(st0[..., 0] - s) <= 32 * u * mag)
    assert np.all(np.abs(st0[..., 1] - m2) <= 64 * u * (m2 + mag ** 2 / 32))
    zs, sts = runs["split3"]
    assert refs.close(zs.view(np.float16), z0.view(np.float16), atol=2e-2, rtol=1e-2)[0] == 0
    s3, m23 = _partials_f64(zs.view(np.float16))
    assert np.all(np.abs(sts[..., 0] - s3) <= 32 * u * mag + 1e-3)
    assert np.all(np.abs(sts[..., 1] - m23) <= 64 * u * (m23 + mag ** 2 / 32) + 1e-3)
    want = refs.r16(refs.add(refs.r16(refs.add_bias(refs.r16(refs.gemm(a, w)), b)), r))
    assert refs.close(z0.view(np.float16), want)[0] == 0


@pytest.mark.parametrize("cfg", [16, 32, 34])
def test_epilogue_builds_store_the_bits_of_the_general_build(lib, gpu, cfg, monkeypatch):
    """The tiles with epilogue builds (the epilogue fixed at compile time: fold + GELU, fold, bias + residual + row
    partials, fp16 bias, bias + GELU, bias + residual, none) store the bits of the build that reads every flag from its
    arguments (SH_GEMM_EPI=0), outputs and row partials alike, on partial tiles in M, and with the fold reading given
    statistics or row partials."""
    import torch
    M, N, K = 520, 768, 448
    a, wh, bh, r = _producer(M, N, K, 170)
    X, WH, BH, R = to_dev(a), to_dev(wh), to_dev(bh), to_dev(r)
    _, w, g, be, b = _problem(M, N, N, 180)
    W, G, BE, Bb = to_dev(w), to_dev(g), to_dev(be), to_dev(b)
    monkeypatch.setenv("SH_GEMM_CFG", str(cfg))
    out = {}
    for gen in ("1", "0"):
        monkeypatch.setenv("SH_GEMM_EPI", gen)
        H = torch.empty((M, N), dtype=torch.float16, device="cuda")
        Pst = _empty32(M, N // 32, 2)
        e = shops.epi(bias=A(BH), residual=A(R), ldr=N, stats_out=A(Pst))
        assert lib.sh_gemm_ex(A(X), A(WH), A(H), M, N, K, K, N, N, None, e) == 0, shops.last_error()
        WP, C, Dd, S = _fold(lib, H, W, G, BE, Bb, M, N, N)
        zs = []
        for act in (0, 1):
            for given in (True, False):
                Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
                e = (shops.epi(bias=A(Dd), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(S), ln_c=A(C)) if given else
                     shops.epi(bias=A(Dd), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(Pst), ln_c=A(C),
                               ln_parts=N // 32, ln_eps=EPS))
                assert lib.sh_gemm_ex(A(H), A(WP), A(Z), M, N, N, N, N, N, None, e) == 0, shops.last_error()
                zs.append(codes(Z))
        for e in (shops.epi(bias=A(BH)), shops.epi(bias=A(BH), act=shops.SH_ACT_GELU),        # fp16 bias builds
                  shops.epi(bias=A(BH), residual=A(R), ldr=N), shops.epi()):                 # and none
            Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
            assert lib.sh_gemm_ex(A(X), A(WH), A(Z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
            zs.append(codes(Z))
        out[gen] = (codes(H), to_np(Pst).view(np.uint32), zs)
    assert np.array_equal(out["1"][0], out["0"][0])
    assert np.array_equal(out["1"][1], out["0"][1])
    for z1, z0 in zip(out["1"][2], out["0"][2]):
        assert np.array_equal(z1, z0)


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [16, 32])
def test_epilogue_builds_give_way_to_the_general_build_past_their_address_range(lib, gpu, cfg, monkeypatch):
    """The epilogue builds address X, W, Z and the residual with 32-bit offsets from scalar bases, so the launch uses
    them only for leading dimensions of X below 2^22 and of Z below 2^24; past that the general build runs. The same
    product with fp16 bias and residual, with X and Z stored compactly, at leading dimensions just inside those limits
    and just past them, stores the same bits every time (and meets the oracle)."""
    import torch
    M, N, K = 2, 192, 64
    rng = np.random.default_rng(7)
    x = rng.standard_normal((M, K)).astype(np.float16)
    w = (rng.standard_normal((K, N)) * 0.1).astype(np.float16)
    b = (rng.standard_normal((1, N)) * 0.1).astype(np.float16)
    r = rng.standard_normal((M, N)).astype(np.float16)
    W, Bb, R = to_dev(w), to_dev(b), to_dev(r)
    monkeypatch.setenv("SH_GEMM_CFG", str(cfg))
    got = []
    for ldx, ldz in ((K, N), ((1 << 22) - 64, (1 << 24) - 192), ((1 << 22) + 64, N), (K, (1 << 24) + 192)):
        X = torch.zeros((M, ldx), dtype=torch.float16, device="cuda")
        X[:, :K] = torch.from_numpy(x).cuda()
        Z = torch.zeros((M, ldz), dtype=torch.float16, device="cuda")
        e = shops.epi(bias=A(Bb), residual=A(R), ldr=N)
        assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, ldx, N, ldz, None, e) == 0, shops.last_error()
        got.append(codes(Z[:, :N].contiguous()))
        del X, Z
    for z in got[1:]:
        assert np.array_equal(z, got[0])
    want = (refs.r16(refs.r16(refs.r16(x.astype(np.float32) @ w.astype(np.float32)) + b.astype(np.float32))
            + r.astype(np.float32)))
    have = got[0].view(np.float16).astype(np.float32)
    assert np.all(np.abs(have - want) <= 2e-2 + 1e-2 * np.abs(want))


@pytest.mark.parametrize("mean,act", [(0.7, 0), (0.7, 1), (60.0, 0)])
def test_fold_from_row_partials(lib, gpu, mean, act):
    """The consumer of row partials (ln_parts = K / 32): H from a GEMM that wrote its partials, then the folded
    GEMM on H against the oracle's LayerNorm -> GEMM -> bias (-> GELU) of the stored H, and against the same
    folded GEMM given sh_row_stats of H (two-pass statistics), which it matches to a few fp16 ulps. mean = 60:
    rows far from zero mean (the partials keep M2 about each block's own mean)."""
    import torch
    M, D, N = 1000, 768, 1536
    a, wh, bh, r = _producer(M, D, 256, 150)
    r = (r.astype(np.float32) + np.float32(mean - 0.7)).astype(np.float16)
    X, WH, BH, R = to_dev(a), to_dev(wh), to_dev(bh), to_dev(r)
    H = torch.empty((M, D), dtype=torch.float16, device="cuda")
    Pst = _empty32(M, D // 32, 2)
    e = shops.epi(bias=A(BH), residual=A(R), ldr=D, stats_out=A(Pst))
    assert lib.sh_gemm_ex(A(X), A(WH), A(H), M, D, 256, 256, D, D, None, e) == 0, shops.last_error()
    h = to_np(H)
    _, w, g, be, b = _problem(M, N, D, 160)
    W, G, BE, Bb = to_dev(w), to_dev(g), to_dev(be), to_dev(b)
    WP, C, Dd, S = _fold(lib, H, W, G, BE, Bb, M, N, D)
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e = shops.epi(bias=A(Dd), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(Pst), ln_c=A(C), ln_parts=D // 32,
                  ln_eps=EPS)
    assert lib.sh_gemm_ex(A(H), A(WP), A(Z), M, N, D, D, N, N, None, e) == 0, shops.last_error()
    Z2 = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e2 = shops.epi(bias=A(Dd), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(S), ln_c=A(C))
    assert lib.sh_gemm_ex(A(H), A(WP), A(Z2), M, N, D, D, N, N, None, e2) == 0, shops.last_error()
    bad, err, _ = refs.close(to_np(Z), _want(h, w, g, be, b, act))
    assert bad == 0, err
    bad, err, _ = refs.close(to_np(Z), to_np(Z2), atol=2e-3, rtol=2e-3)
    assert bad == 0, err
    # the same partials 8 bytes into a buffer (8-byte, not 16-byte aligned): read 8 bytes at a time, the same bits
    Pst8 = _empty32(M * (D // 32) * 2 + 2)
    Pst8[2:].copy_(Pst.reshape(-1))
    assert (A(Pst8) + 8) % 16 == 8
    Z8 = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e8 = shops.epi(bias=A(Dd), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(Pst8) + 8, ln_c=A(C),
                   ln_parts=D // 32, ln_eps=EPS)
    assert lib.sh_gemm_ex(A(H), A(WP), A(Z8), M, N, D, D, N, N, None, e8) == 0, shops.last_error()
    assert np.array_equal(codes(Z8), codes(Z))
    e4 = shops.epi(bias=A(Dd), bias_fmt=shops.SH_BIAS_FP32, act=act, ln_stats=A(Pst8) + 4, ln_c=A(C),
                   ln_parts=D // 32, ln_eps=EPS)
    assert lib.sh_gemm_ex(A(H), A(WP), A(Z8), M, N, D, D, N, N, None, e4) == -1          # 4-byte aligned: refused


def test_row_partials_argument_errors(lib, gpu):
    import torch
    M, N, K = 256, 768, 256
    X = to_dev(data.normal((M, K), 1))
    W = to_dev(data.normal((K, N), 2))
    W584 = to_dev(data.normal((K, 584), 3))
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    St = _empty32(M, N // 32 + 1, 2)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, shops.epi(stats_out=A(St) + 4)) == -1   # alignment
    assert lib.sh_gemm_ex(A(X), A(W584), A(Z), M, 584, K, K, 584, 584, None, shops.epi(stats_out=A(St))) == -1  # N % 32
    S, C, D = _empty32(M, 8, 2), _empty32(N), _empty32(N)
    e = shops.epi(bias=A(D), bias_fmt=shops.SH_BIAS_FP32, ln_stats=A(S), ln_c=A(C), ln_parts=4, ln_eps=EPS)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, e) == -1                                # 4 x 32 != K
