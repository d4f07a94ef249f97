"""sh_gemm / sh_gemm_splitk / sh_gemm_mesh / sh_gemm_ex on the GPU against the numpy oracle.

Cases follow the reference's GEMM tests: run.py DEFAULT_GEMM shapes and fills (run.py:54-56, 87-93; small
integers, exact), REAL_DATA fills (gemm/main.c:18-20), the gemm_seq pattern with strided head slices
(gemm_seq/main.c:29-50), the SUMMA known answer (examples/gemm1024_summa.mlir:5), and the BASELINE config-1/2
shapes. Tolerance for real-valued data: |got - want| <= 2e-2 + 1e-2 |want| against the fp32 product.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import K2_CFGS, K5_CFGS, KG2_CFGS, REGSTAGED_CFGS, TILE_CFGS, codes, to_dev, to_np
from oracle import lcg, refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
NUM_TILE_CFGS = TILE_CFGS      # entries of the GEMM tile table (g_cfgs in sh_gemm.hip)
A = shops.addr


def _run_gemm(lib, x, w, z0=None, cfg=None, M=None, N=None, K=None, splits=None):
    import torch
    M, K = x.shape
    N = w.shape[1]
    X, W = to_dev(x), to_dev(w)
    Z = to_dev(z0) if z0 is not None else torch.zeros((M, N), dtype=torch.float16, device="cuda")
    if splits is None:
        rc = lib.sh_gemm(A(X), A(W), A(Z), M, N, K, K, N, N, cfg, shops.SH_ALL)
    else:
        rc = lib.sh_gemm_splitk(A(X), A(W), A(Z), M, N, K, K, N, N, cfg, splits, shops.SH_ALL)
    assert rc == 0, shops.last_error()
    return X, W, Z


def _parse(shape: str):
    dims, _, rest = shape.partition(":")
    M, N, K = (int(v) for v in dims.split("x"))
    o = rest.split(",") if rest else []
    tm, tn, tk = (int(v) for v in (o + ["0", "0", "0"])[:3])
    pipe = int(o[3]) if len(o) > 3 else 1
    acc = int(o[4]) if len(o) > 4 else 0
    return M, N, K, shops.cfg(tm, tn, tk, pipe, acc), acc


DEFAULT_GEMM = ["256x256x256", "256x768x192:256,256,192", "512x768x768:256,256,256", "256x256x256:256,256,256,0",
                "256x256x512:256,256,256,1,1", "1024x768x768:256,256,256,1,0", "1024x3072x768:256,256,256,1,0"]


@pytest.mark.parametrize("shape", DEFAULT_GEMM)
def test_reference_default_shapes_exact(lib, gpu, shape):
    M, N, K, cfg, acc = _parse(shape)
    x = lcg.fill_fp16(M, K, 1, -1, 1)
    w = lcg.fill_fp16(K, N, 2, -2, 2)
    z0 = lcg.fill_fp16(M, N, 3, 3 if acc else 0, 3 if acc else 0)
    X, W, Z = _run_gemm(lib, x, w, z0, cfg)
    want = refs.gemm(x, w, z0 if acc else None)
    assert np.array_equal(to_np(Z).astype(np.float32), want)          # integers below 2048: exact in fp16
    with shops.capture() as cap:
        bad = lib.sh_test_check_gemm(A(X), A(W), A(Z), M, N, K, K, N, N, 256, 0.5, 3.0 if acc else 0.0, b"[gemm]")
    assert bad == 0 and "bad=0" in cap.text and "PASS" in cap.text


def test_real_data_fills(lib, gpu):
    M, N, K = 512, 768, 768
    x = lcg.fill_fp16(M, K, 1, 0, 64, 1 / 4096)
    w = lcg.fill_fp16(K, N, 2, -16, 16, 0.125)
    _, _, Z = _run_gemm(lib, x, w)
    bad, err, _ = refs.close(to_np(Z), refs.gemm(x, w))
    assert bad == 0, err


@pytest.mark.parametrize("K", [136, 192])
@pytest.mark.parametrize("cfg_index", range(NUM_TILE_CFGS))
def test_every_tile_config(lib, gpu, cfg_index, K, monkeypatch):
    """Each compiled tile shape on a problem with partial tiles in M and N; K = 136 has a K tail (only the
    general kernels take it), K = 192 is a multiple of 64 (the direct-to-LDS kernels take it)."""
    monkeypatch.setenv("SH_GEMM_CFG", str(cfg_index))
    M, N = 328, 200
    x = data.normal((M, K), 11)
    w = data.normal((K, N), 12, std=1 / np.sqrt(K))
    import torch
    X, W = to_dev(x), to_dev(w)
    Z = torch.full((M + 3, 208), 7.0, dtype=torch.float16, device="cuda")           # ldz = 208 > N, poison
    rc = lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, 208, None, None)
    assert rc == 0, shops.last_error()
    z = to_np(Z)
    bad, err, _ = refs.close(z[:M, :N], refs.gemm(x, w))
    assert bad == 0, err
    assert (z[:M, N:] == 7.0).all() and (z[M:] == 7.0).all()                       # nothing outside the view


def test_unsplit_tile_configs_store_identical_bits(lib, gpu, monkeypatch):
    """Unsplit tile configurations of one kernel family accumulate K in the same order with the same MFMA
    operand layout, so the choice between them (the library times them once per shape) never changes a bit."""
    import torch
    M, N, K = 520, 392, 448
    x, w = data.normal((M, K), 21), data.normal((K, N), 22, std=1 / np.sqrt(K))
    X, W = to_dev(x), to_dev(w)
    outs = []
    for cfg_index in range(NUM_TILE_CFGS):
        monkeypatch.setenv("SH_GEMM_CFG", str(cfg_index))
        Z = torch.zeros((M, N), dtype=torch.float16, device="cuda")
        assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, None) == 0, shops.last_error()
        outs.append(to_np(Z).view(np.uint16))
    # the direct-to-LDS kernels the cost model and the one-time timing choose between (k_gemm2 and k_gemm5: 64-row
    # to 256-row tiles, 64-k and 32-k slices, LDS-staged or register epilogue; a W^T configuration forced on a W
    # call runs the model's choice) agree bit for bit; so do the register-staged fallbacks among themselves
    direct = [i for i in range(NUM_TILE_CFGS) if i not in REGSTAGED_CFGS]
    for group in (direct, list(REGSTAGED_CFGS)):
        for i in group:
            assert (outs[i] == outs[group[0]]).all(), f"config {i} differs from config {group[0]}"
    for i in (REGSTAGED_CFGS[0], direct[0]):
        assert refs.close(outs[i].view(np.float16), refs.gemm(x, w))[0] == 0


REG_EPILOGUE_CFGS = K5_CFGS   # register-epilogue tiles (W layout)


@pytest.mark.parametrize("K", [64, 448])
def test_register_epilogue_configs_with_residual(lib, gpu, K, monkeypatch):
    """Register-epilogue tiles (k_gemm5: each wavefront stores its block through its own LDS slots as whole
    row segments and add the residual there) on partial tiles in M and N with ldz > N, bias + GELU and
    bias + residual epilogues: bit-identical to configuration 6 (LDS-staged epilogue of the whole tile), rows
    sampled against the oracle, nothing written outside the view. K = 64 is a single slice."""
    import torch
    M, N = 1000, 584
    x = data.normal((M, K), 61)
    w = data.normal((K, N), 62, std=1 / np.sqrt(K))
    b = data.normal((1, N), 63, std=0.3)
    r = data.normal((M, N), 64)
    X, W, Bb, R = to_dev(x), to_dev(w), to_dev(b), to_dev(r)
    rows = np.array([0, 1, 31, 32, 127, 128, 511, 999])
    for epi in ("gelu", "res"):
        e = (shops.epi(bias=A(Bb), act=shops.SH_ACT_GELU) if epi == "gelu"
             else shops.epi(bias=A(Bb), residual=A(R), ldr=N))
        outs = {}
        for cfg in (6,) + REG_EPILOGUE_CFGS:
            monkeypatch.setenv("SH_GEMM_CFG", str(cfg))
            Z = torch.full((M, N + 8), 7.0, dtype=torch.float16, device="cuda")
            assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N + 8, None, e) == 0, (cfg, shops.last_error())
            assert (to_np(Z)[:, N:] == 7.0).all(), cfg
            outs[cfg] = codes(Z)[:, :N]
        for cfg in REG_EPILOGUE_CFGS:
            assert np.array_equal(outs[cfg], outs[6]), (epi, cfg, int((outs[cfg] != outs[6]).sum()))
        zs = refs.r16(refs.add_bias(refs.r16(refs.gemm(x[rows], w)), b))
        want = refs.r16(refs.gelu(zs)) if epi == "gelu" else refs.r16(refs.add(zs, r[rows]))
        bad, err, _ = refs.close(outs[6][rows].view(np.float16), want)
        assert bad == 0, (epi, err)


def test_scalar_path_unaligned_views(lib, gpu):
    """Odd N and K, and operands starting one element into their buffers (no 16-byte alignment)."""
    import torch
    M, N, K = 70, 45, 37
    x = data.normal((M, K + 1), 21)
    w = data.normal((K + 1, N + 3), 22, std=0.2)
    X, W = to_dev(x), to_dev(w)
    Z = torch.zeros((M, N + 2), dtype=torch.float16, device="cuda")
    rc = lib.sh_gemm_ex(A(X, 1), A(W, 1), A(Z, 1), M, N, K, K + 1, N + 3, N + 2, None, None)
    assert rc == 0, shops.last_error()
    want = refs.gemm(x[:, 1:], w[:K, 1:N + 1])
    bad, err, _ = refs.close(to_np(Z)[:, 1:N + 1], want)
    assert bad == 0, err


def test_fused_epilogue_bias_gelu_residual(lib, gpu):
    import torch
    M, N, K = 384, 576, 320
    x = data.normal((M, K), 31)
    w = data.normal((K, N), 32, std=1 / np.sqrt(K))
    b32 = (np.random.default_rng(33).random((1, N), dtype=np.float32) * 0.2 - 0.1)
    r = data.normal((M, N), 34)
    X, W, R = to_dev(x), to_dev(w), to_dev(r)
    B32 = torch.from_numpy(b32).cuda()
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e = shops.epi(bias=A(B32), bias_fmt=shops.SH_BIAS_FP32, act=shops.SH_ACT_GELU, residual=A(R), ldr=N)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    want = refs.r16(refs.gelu(refs.gemm(x, w) + b32)) + r.astype(np.float32)
    bad, err, _ = refs.close(to_np(Z), want)
    assert bad == 0, err
    # residual aliasing the output (z = z + act(XW + b)), fp16 bias, split into 3
    Z2 = to_dev(r)
    B16 = to_dev(b32.astype(np.float16))
    e = shops.epi(bias=A(B16), bias_fmt=shops.SH_BIAS_FP16, residual=A(Z2), ldr=N, splits=3)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z2), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    want = refs.gemm(x, w) + b32.astype(np.float16).astype(np.float32) + r.astype(np.float32)
    bad, err, _ = refs.close(to_np(Z2), want)
    assert bad == 0, err


@pytest.mark.parametrize("act,accumulate", [(shops.SH_ACT_GELU, 0), (shops.SH_ACT_NONE, 1)])
def test_fused_epilogue_is_the_library_sequence_bitwise(lib, gpu, act, accumulate):
    """sh_gemm_ex(bias fp16 [+GELU] + residual) stores exactly what the reference's unfused sequence stores:
    sh_gemm (Z = or Z +=) -> sh_add_bias -> [sh_gelu] -> sh_add (siglip.py:150-168 op order), bit for bit."""
    import torch
    M, N, K = 320, 448, 256
    x, w = data.normal((M, K), 41), data.normal((K, N), 42, std=1 / np.sqrt(K))
    b16, r, z0 = data.normal((1, N), 43, std=0.5), data.normal((M, N), 44), data.normal((M, N), 45)
    X, W, B16, R = to_dev(x), to_dev(w), to_dev(b16), to_dev(r)
    Z1, Z2 = to_dev(z0), to_dev(z0)
    c = shops.cfg(64, 64, 64, accumulate=accumulate)          # tiles that divide M, N, K (sh_gemm.inc.c:60-63)
    e = shops.epi(bias=A(B16), act=act, residual=A(R), ldr=N)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z1), M, N, K, K, N, N, c, e) == 0, shops.last_error()
    assert lib.sh_gemm(A(X), A(W), A(Z2), M, N, K, K, N, N, c, shops.SH_ALL) == 0
    lib.sh_add_bias(A(Z2), A(Z2), A(B16), M, N, N, shops.SH_ALL)
    if act == shops.SH_ACT_GELU:
        lib.sh_gelu(A(Z2), A(Z2), M, N, N, shops.SH_ALL)
    lib.sh_add(A(Z2), A(Z2), A(R), M, N, N, shops.SH_ALL)
    torch.cuda.synchronize()
    z1, z2 = to_np(Z1).view(np.uint16), to_np(Z2).view(np.uint16)
    bad = np.argwhere(z1 != z2)
    assert len(bad) == 0, f"{len(bad)} differ, e.g. " + ", ".join(f"{tuple(ix)}: {z1[tuple(ix)]:04x} vs {z2[tuple(ix)]:04x}" for ix in bad[:6])


# (bias format, act, residual, accumulate): every branch of the epilogue chain, including the register epilogue's
# two load paths (fp16 bias / residual in one batch; z_old or an fp32 bias per row and column block)
EPI_CASES = [(shops.SH_BIAS_FP16, shops.SH_ACT_GELU, True, 0), (shops.SH_BIAS_FP32, shops.SH_ACT_NONE, True, 1),
             (shops.SH_BIAS_FP32, shops.SH_ACT_GELU, False, 0), (None, shops.SH_ACT_NONE, False, 1),
             (None, shops.SH_ACT_NONE, False, 0)]


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("case", range(len(EPI_CASES)))
def test_epilogue_chain_same_bits_on_every_tile(lib, gpu, monkeypatch, case, splits):
    """Each epilogue combination on partial tiles (M, N not multiples of any tile), on the LDS-staged and the
    register-epilogue tile configurations (k_gemm2 256x256 and its 64x64, 64x128, 128x64 tiles; every k_gemm5
    tile: register epilogue, 32- and 64-k slices): every configuration stores the same bits (split or not),
    nothing outside the output view changes, and the result is within tolerance of the oracle's unfused
    sequence."""
    import torch
    bias_fmt, act, res, accumulate = EPI_CASES[case]
    M, N, K, ldz = 328, 200, 192, 208
    x, w = data.normal((M, K), 51), data.normal((K, N), 52, std=1 / np.sqrt(K))
    b32 = data.normal((1, N), 53, std=0.3).astype(np.float32)
    r, z0 = data.normal((M, N), 54), data.normal((M, N), 55)
    X, W, R = to_dev(x), to_dev(w), to_dev(r)
    bias = None
    if bias_fmt == shops.SH_BIAS_FP32:
        bias = torch.from_numpy(b32).cuda()
    elif bias_fmt == shops.SH_BIAS_FP16:
        bias = to_dev(b32.astype(np.float16))
    outs = {}
    for cfg_index in (K2_CFGS[0],) + K5_CFGS + K2_CFGS[-3:]:
        monkeypatch.setenv("SH_GEMM_CFG", str(cfg_index))
        Z = torch.full((M + 3, ldz), 7.0, dtype=torch.float16, device="cuda")
        Z[:M, :N] = to_dev(z0)
        e = shops.epi(bias=A(bias) if bias is not None else 0, bias_fmt=bias_fmt or 0, act=act,
                      residual=A(R) if res else 0, ldr=N if res else 0, splits=splits)
        c = shops.cfg(accumulate=accumulate)
        assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, ldz, c, e) == 0, shops.last_error()
        z = to_np(Z)
        assert (z[:M, N:] == 7.0).all() and (z[M:] == 7.0).all(), f"config {cfg_index} wrote outside the view"
        outs[cfg_index] = z[:M, :N].view(np.uint16).copy()
    for cfg_index, o in outs.items():
        assert (o == outs[K2_CFGS[0]]).all(), f"config {cfg_index} differs from config {K2_CFGS[0]} in {(o != outs[K2_CFGS[0]]).sum()} elements"
    # the reference's unfused order: Z (+)= XW, + bias, GELU, + residual, each stored in fp16
    want = refs.gemm(x, w, z0 if accumulate else None)
    if bias is not None:
        bb = b32 if bias_fmt == shops.SH_BIAS_FP32 else b32.astype(np.float16).astype(np.float32)
        want = refs.r16(want + bb)
    if act == shops.SH_ACT_GELU:
        want = refs.r16(refs.gelu(want))
    if res:
        want = want + r.astype(np.float32)
    bad, err, _ = refs.close(outs[K2_CFGS[0]].view(np.float16), want)
    assert bad == 0, err


def test_splitk_matches_and_is_deterministic(lib, gpu):
    """BASELINE config 2 FFN-down: M=256, K=3072, N=768, split-K = 4."""
    M, N, K = 256, 768, 3072
    x = data.uniform(M, K, 41)
    w = (data.uniform(K, N, 42).astype(np.float32) / np.sqrt(K)).astype(np.float16)
    _, _, Z1 = _run_gemm(lib, x, w, splits=4)
    _, _, Z2 = _run_gemm(lib, x, w, splits=4)
    _, _, Z0 = _run_gemm(lib, x, w, splits=1)
    want = refs.gemm(x, w)
    for Z in (Z1, Z0):
        bad, err, _ = refs.close(to_np(Z), want)
        assert bad == 0, err
    assert np.array_equal(codes(Z1), codes(Z2))
    # accumulate through split-K: Z = Z0 + XW
    z0 = data.normal((M, N), 43)
    _, _, Z3 = _run_gemm(lib, x, w, z0=z0, cfg=shops.cfg(accumulate=1), splits=3)
    bad, err, _ = refs.close(to_np(Z3), want + z0.astype(np.float32))
    assert bad == 0, err



def test_splitk_on_two_streams_keeps_partials_apart(lib, gpu):
    """Split-K calls alternating on two torch streams with no synchronisation between them: each stream has its
    own partial workspace, so every result equals the same call run alone, bit for bit, and the fp32 product
    within tolerance. The two streams run different shapes and split counts, so a shared workspace would mix
    their partials."""
    import torch
    shapes = [(256, 768, 3072, 4), (512, 512, 2048, 3)]
    ins = []
    for si, (M, N, K, _) in enumerate(shapes):
        x = data.uniform(M, K, 51 + si)
        w = (data.uniform(K, N, 61 + si).astype(np.float32) / np.sqrt(K)).astype(np.float16)
        ins.append((x, w))
    alone = [codes(_run_gemm(lib, x, w, splits=s)[2]) for (_, _, _, s), (x, w) in zip(shapes, ins)]
    dev = [(to_dev(x), to_dev(w)) for x, w in ins]
    outs = [[torch.zeros((M, N), dtype=torch.float16, device="cuda") for _ in range(3)] for M, N, _, _ in shapes]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    prev = lib.sh_get_stream()
    torch.cuda.synchronize()
    try:
        for rep in range(3):
            for si, ((M, N, K, s), (X, W)) in enumerate(zip(shapes, dev)):
                lib.sh_set_stream(streams[si].cuda_stream)
                rc = lib.sh_gemm_splitk(A(X), A(W), A(outs[si][rep]), M, N, K, K, N, N, None, s, shops.SH_ALL)
                assert rc == 0, shops.last_error()
    finally:
        lib.sh_set_stream(prev)
    torch.cuda.synchronize()
    for si in range(len(shapes)):
        for rep in range(3):
            assert np.array_equal(codes(outs[si][rep]), alone[si]), (si, rep)
        bad, err, _ = refs.close(to_np(outs[si][0]), refs.gemm(*ins[si]))
        assert bad == 0, err
    # each stream holds its own workspace until sh_stream_release frees it; a later call on it allocates again
    for st in streams:
        assert lib.sh_stream_workspace_bytes(st.cuda_stream) >= 64 << 20
    free0 = torch.cuda.mem_get_info()[0]
    for st in streams:
        assert lib.sh_stream_release(st.cuda_stream) == 0, shops.last_error()
        assert lib.sh_stream_workspace_bytes(st.cuda_stream) == 0
    assert torch.cuda.mem_get_info()[0] >= free0 + (100 << 20)               # two 64 MiB workspaces returned
    assert lib.sh_stream_release(streams[0].cuda_stream) == 0                # nothing held: nothing to do
    (M, N, K, s), (X, W) = shapes[0], dev[0]
    Z = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    try:
        lib.sh_set_stream(streams[0].cuda_stream)
        assert lib.sh_gemm_splitk(A(X), A(W), A(Z), M, N, K, K, N, N, None, s, shops.SH_ALL) == 0, shops.last_error()
    finally:
        lib.sh_set_stream(prev)
    torch.cuda.synchronize()
    assert np.array_equal(codes(Z), alone[0])

_ORDER_CHILD = r"""
import os, sys
import numpy as np, torch
from softhier_mlir_amd import shops
lib = shops.load(); lib.sh_init()
M, N, K = 1000, 1128, 768                     # 8 x 6 tiles of 128 x 192 (the last row and column partial)
g = torch.Generator(device="cuda").manual_seed(5)
x = torch.randn((M, K), dtype=torch.float16, device="cuda", generator=g)
w = (torch.randn((K, N), dtype=torch.float16, device="cuda", generator=g) * 0.04).contiguous()
b = torch.randn((1, N), dtype=torch.float16, device="cuda", generator=g)
r = torch.randn((M, N), dtype=torch.float16, device="cuda", generator=g)
z = torch.zeros((M, N), dtype=torch.float16, device="cuda")
A = shops.addr
e = shops.epi(bias=A(b), residual=A(r), ldr=N)
assert lib.sh_gemm_ex(A(x), A(w), A(z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
torch.cuda.synchronize()
np.save(sys.argv[1], z.cpu().numpy().view(np.uint16))
"""


def test_tile_order_bands_store_identical_bits(lib, gpu, tmp_path):
    """The tile order (row-major, or bands of SH_GEMM_GROUP tile rows taken column by column; read once per process,
    so each setting runs in its own child process, one after another) only moves tiles between workgroups: bands of
    1 (row-major), 3 (a short last band on this 8-row grid) and 8 (the default) store the same bits, with a
    128x192 tile, bias and residual."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    outs = {}
    for band in (1, 3, 8):
        env = dict(os.environ, SH_GEMM_GROUP=str(band), SH_GEMM_CFG=str(KG2_CFGS[1]), PYTHONPATH=root)
        f = tmp_path / f"z{band}.npy"
        rc = subprocess.run([sys.executable, "-c", _ORDER_CHILD, str(f)], env=env, cwd=root, timeout=110,
                            capture_output=True, text=True)
        assert rc.returncode == 0, (band, rc.stderr[-2000:])
        outs[band] = np.load(f)
    assert np.array_equal(outs[1], outs[3]) and np.array_equal(outs[1], outs[8])




@pytest.mark.parametrize("M,N,K", [(1000, 760, 768), (520, 768, 3072), (8192, 768, 3072), (300, 256, 128)])
def test_in_workgroup_split_k_stores_the_two_partial_bits(lib, gpu, monkeypatch, M, N, K):
    """A request for two K ranges with K % 128 == 0 runs as one workgroup per tile whose two wavefront groups each
    take one range and add their fp32 accumulators in LDS (k_gemm5 KG = 2). Its outputs are the bits of the
    two-partial path on the same tile (SH_GEMM_KG=0: fp32 partials in HBM, the reduction adds first + second; a plan
    on a register-staged tile, which accumulates in another order, keeps that path) for every epilogue:
    none, bias + GELU, bias + residual with accumulate, the LayerNorm fold with GELU, and bias + residual writing
    row partials (those match float64 sums over the stored output); both tiles with the variant agree, ragged M
    and N included, nothing is written outside the view (ldz = N + 8), and sampled rows match the oracle."""
    import torch
    x = data.normal((M, K), 171)
    w = data.normal((K, N), 172, std=1 / np.sqrt(K))
    b = data.normal((1, N), 173, std=0.3)
    r = data.normal((M, N), 174)
    z0 = data.normal((M, N), 175)
    g = (1.0 + data.normal((1, K), 176, std=0.2)).astype(np.float16)
    be = data.normal((1, K), 177, std=0.2)
    X, W, Bb, R, G, BE = (to_dev(v) for v in (x, w, b, r, g, be))
    f32 = dict(dtype=torch.float32, device="cuda")
    WP, C, D, S = torch.empty((K, N), dtype=torch.float16, device="cuda"), torch.empty(N, **f32), torch.empty(N, **f32), torch.empty((M, 2), **f32)
    lib.sh_ln_fold(A(WP), A(C), A(D), A(W), A(G), A(BE), A(Bb), K, N, N, N)
    lib.sh_row_stats(A(S), A(X), M, K, K, 1e-6)
    assert shops.last_error()[0] == 0, shops.last_error()
    P = N // 32
    GELU, FP32 = shops.SH_ACT_GELU, shops.SH_BIAS_FP32
    cases = {
        "plain": (W, lambda st: shops.epi(splits=2), None),
        "gelu": (W, lambda st: shops.epi(bias=A(Bb), act=GELU, splits=2), None),
        "res_acc": (W, lambda st: shops.epi(bias=A(Bb), residual=A(R), ldr=N, splits=2), shops.cfg(accumulate=1)),
        "lnfold": (WP, lambda st: shops.epi(bias=A(D), bias_fmt=FP32, act=GELU, ln_stats=A(S), ln_c=A(C), splits=2), None),
    }
    if N % 32 == 0:
        cases["stats"] = (W, lambda st: shops.epi(bias=A(Bb), residual=A(R), ldr=N, stats_out=A(st), splits=2), None)

    def run(name, kg, cfg_index):
        Wm, mk, gcfg = cases[name]
        monkeypatch.setenv("SH_GEMM_KG", str(kg))
        if cfg_index is None:
            monkeypatch.delenv("SH_GEMM_CFG", raising=False)
        else:
            monkeypatch.setenv("SH_GEMM_CFG", str(cfg_index))
        Z = torch.full((M, N + 8), 7.0, dtype=torch.float16, device="cuda")
        if gcfg is not None:
            Z[:, :N] = to_dev(z0)
        St = torch.zeros((M, max(P, 1), 2), **f32)
        rc = lib.sh_gemm_ex(A(X), A(Wm), A(Z), M, N, K, K, N, N + 8, gcfg, mk(St))
        assert rc == 0, (name, kg, cfg_index, shops.last_error())
        assert (to_np(Z)[:, N:] == 7.0).all(), (name, kg, cfg_index)
        return codes(Z)[:, :N], to_np(St)

    rows = np.array([0, 1, 31, 127, 128, M // 2, M - 1])
    for name in cases:
        outs = []
        for cfg_index in (None,) + KG2_CFGS:
            want, _ = run(name, 0, cfg_index)
            got, st = run(name, 1, cfg_index)
            assert np.array_equal(got, want), (name, cfg_index, int((got != want).sum()))
            outs.append(got)
            if name == "stats":
                zf = got.view(np.float16).astype(np.float64).reshape(M, P, 32)
                s = zf.sum(2)
                m2 = ((zf - s[..., None] / 32) ** 2).sum(2)
                mag, u = np.abs(zf).sum(2), 2.0 ** -24
                assert np.all(np.abs(st[..., 0] - s) <= 32 * u * mag)
                assert np.all(np.abs(st[..., 1] - m2) <= 64 * u * (m2 + mag ** 2 / 32))
        assert np.array_equal(outs[1], outs[2]), name
        if name == "plain":
            bad, err, _ = refs.close(want[rows].view(np.float16), refs.gemm(x[rows], w))
            assert bad == 0, err


def test_mesh_known_answer_and_lcg(lib, gpu):
    import torch
    M = N = K = 1024
    X = torch.ones((M, K), dtype=torch.float16, device="cuda")
    W = torch.full((K, N), 1 / 1024, dtype=torch.float16, device="cuda")
    Z = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    c = shops.cfg(256, 256, 256, 1, 0)
    assert lib.sh_gemm_mesh(A(X), A(W), A(Z), M, N, K, K, N, N, c) == 0, shops.last_error()
    assert (to_np(Z) == 1.0).all()                                   # examples/gemm1024_summa.mlir:5
    x = data.uniform(M, K, 51)
    w = (data.uniform(K, N, 52).astype(np.float32) / 32).astype(np.float16)
    Xd, Wd = to_dev(x), to_dev(w)
    assert lib.sh_gemm_mesh(A(Xd), A(Wd), A(Z), M, N, K, K, N, N, c) == 0
    bad, err, _ = refs.close(to_np(Z), refs.gemm(x, w))
    assert bad == 0, err


def test_gemm_seq_strided_head_slices(lib, gpu):
    """gemm_seq/main.c: mixed tiles back to back, 64-column head slices of 768-wide W/Z (ld = 768), and the
    in-place softmax(P) . V slice on real data; the rest of the sliced Z keeps its poison."""
    import torch
    f = lcg.fill_fp16
    xa, wa = f(256, 64, 1, -1, 1), f(64, 256, 2, -2, 2)
    xb, wb = f(256, 256, 3, -1, 1), f(256, 64, 4, -2, 2)
    xd, wd, zd = f(256, 256, 7, -1, 1), f(256, 768, 8, -2, 2), f(256, 768, 9, 7, 7)
    xe, we = f(256, 256, 10, -32, 32, 0.125), f(256, 768, 11, -16, 16, 0.125)
    Xa, Wa, Za = to_dev(xa), to_dev(wa), torch.zeros((256, 256), dtype=torch.float16, device="cuda")
    Xb, Wb, Zb = to_dev(xb), to_dev(wb), torch.zeros((256, 64), dtype=torch.float16, device="cuda")
    Xd, Wd, Zd = to_dev(xd), to_dev(wd), to_dev(zd)
    Xe, We, Ze = to_dev(xe), to_dev(we), torch.zeros((256, 768), dtype=torch.float16, device="cuda")
    a = shops.cfg(256, 256, 64, 1)
    b = shops.cfg(256, 64, 256, 1)
    lib.sh_softmax_rows(A(Xe), A(Xe), 256, 256, 256, 0.125, 0)
    assert lib.sh_gemm(A(Xa), A(Wa), A(Za), 256, 256, 64, 64, 256, 256, a, 0) == 0
    assert lib.sh_gemm(A(Xb), A(Wb), A(Zb), 256, 64, 256, 256, 64, 64, b, 0) == 0
    assert lib.sh_gemm(A(Xd), A(Wd, 6 * 64), A(Zd, 6 * 64), 256, 64, 256, 256, 768, 768, b, 0) == 0
    assert lib.sh_gemm(A(Xe), A(We), A(Ze), 256, 64, 256, 256, 768, 768, b, 0) == 0
    assert np.array_equal(to_np(Za).astype(np.float32), refs.gemm(xa, wa))
    assert np.array_equal(to_np(Zb).astype(np.float32), refs.gemm(xb, wb))
    zd_got = to_np(Zd)
    assert np.array_equal(zd_got[:, 384:448].astype(np.float32), refs.gemm(xd, wd[:, 384:448]))
    assert (np.delete(zd_got, np.s_[384:448], axis=1) == 7.0).all()
    p = refs.r16(refs.softmax(xe, 0.125))
    bad, err, _ = refs.close(to_np(Ze)[:, :64], refs.gemm(p.astype(np.float16), we[:, :64]))
    assert bad == 0, err
    assert (to_np(Ze)[:, 64:] == 0).all()


@pytest.mark.parametrize("M,N,K,epi", [(256, 2304, 768, "bias"), (256, 3072, 768, "bias_gelu"), (256, 768, 3072, "splitk4")])
def test_baseline_config2_shapes(lib, gpu, M, N, K, epi):
    import torch
    x = data.uniform(M, K, 61)
    w = (data.uniform(K, N, 62).astype(np.float32) / np.sqrt(K)).astype(np.float16)
    b32 = (data.uniform(1, N, 63).astype(np.float32) * 0.1)
    X, W = to_dev(x), to_dev(w)
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    if epi == "splitk4":
        assert lib.sh_gemm_splitk(A(X), A(W), A(Z), M, N, K, K, N, N, None, 4, shops.SH_ALL) == 0
        want = refs.gemm(x, w)
    else:
        # library call sequence of the reference: sh_gemm then sh_add_bias (fp16 bias row) [then sh_gelu]
        B16 = to_dev(b32.astype(np.float16))
        assert lib.sh_gemm(A(X), A(W), A(Z), M, N, K, K, N, N, shops.cfg(256, 256, 256), shops.SH_ALL) == 0
        lib.sh_add_bias(A(Z), A(Z), A(B16), M, N, N, shops.SH_ALL)
        want = refs.r16(refs.gemm(x, w)) + b32.astype(np.float16).astype(np.float32)
        if epi == "bias_gelu":
            lib.sh_gelu(A(Z), A(Z), M, N, N, shops.SH_ALL)
            want = refs.gelu(refs.r16(want))
    bad, err, _ = refs.close(to_np(Z), want)
    assert bad == 0, err


@pytest.mark.parametrize("M,N,K,act,splits", [(256, 2304, 768, 0, 1), (256, 3072, 768, 1, 1), (256, 768, 3072, 0, 4)])
def test_baseline_config2_fp32_bias_epilogue(lib, gpu, M, N, K, act, splits):
    """BASELINE config 2 with its fp32 bias row (uniform [-0.1, 0.1]) applied in the GEMM epilogue: QKV + bias,
    FFN-up + bias + tanh-GELU, FFN-down split-K 4 + bias. The epilogue rounds where the unfused sequence stores:
    r16(r16(X W) + b) [then GELU of that fp16 value]."""
    import torch
    x = data.uniform(M, K, 61)
    w = (data.uniform(K, N, 62).astype(np.float32) / np.sqrt(K)).astype(np.float16)
    b32 = (data.uniform(1, N, 63).astype(np.float32) * np.float32(0.1))
    X, W, Bf = to_dev(x), to_dev(w), torch.from_numpy(b32).to("cuda")
    Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
    e = shops.epi(bias=A(Bf), bias_fmt=shops.SH_BIAS_FP32, act=shops.SH_ACT_GELU if act else shops.SH_ACT_NONE, splits=splits)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, e) == 0, shops.last_error()
    want = refs.r16(refs.r16(refs.gemm(x, w)) + b32)
    if act:
        want = refs.gelu(want)
    got = to_np(Z)
    bad, err, _ = refs.close(got, want)
    assert bad == 0, err
    # the bias is really applied: the same call without it differs by the bias row (within fp16 rounding)
    Z0 = torch.empty_like(Z)
    e0 = shops.epi(splits=splits)
    assert lib.sh_gemm_ex(A(X), A(W), A(Z0), M, N, K, K, N, N, None, e0) == 0, shops.last_error()
    if not act:
        d = got.astype(np.float32) - to_np(Z0).astype(np.float32)
        assert np.abs(d - b32).max() <= 2e-3 * (1 + np.abs(got.astype(np.float32)).max())


def test_config1_single_gemm(lib, gpu):
    x = data.uniform(256, 256, 1)
    w = data.uniform(256, 256, 2)
    _, _, Z = _run_gemm(lib, x, w)
    bad, err, _ = refs.close(to_np(Z), refs.gemm(x, w))
    assert bad == 0, err


def test_large_encoder_shape_property(lib, gpu):
    """M = 8192 (B = 32 rows of the encoder): known answers at full size. W = I (identity blocks) reproduces X
    exactly; a W whose column j holds the constant j + 1 (a row-sum W) gives (j + 1) times each row's sum,
    checked against the float64 row sums within the fp16 tolerance (sums of up to 768 fp32 products)."""
    import torch
    M, K = 8192, 768
    x = data.normal((M, K), 71)
    X = to_dev(x)
    I = torch.eye(K, dtype=torch.float16, device="cuda")
    Z = torch.empty((M, K), dtype=torch.float16, device="cuda")
    assert lib.sh_gemm(A(X), A(I), A(Z), M, K, K, K, K, K, None, shops.SH_ALL) == 0
    assert np.array_equal(codes(Z), x.view(np.uint16))
    N = 256
    Ws = torch.arange(1, N + 1, dtype=torch.float16, device="cuda").repeat(K, 1).contiguous()
    Zs = torch.empty((M, N), dtype=torch.float16, device="cuda")
    assert lib.sh_gemm(A(X), A(Ws), A(Zs), M, N, K, K, N, N, None, shops.SH_ALL) == 0
    rs = x.astype(np.float64).sum(axis=1)
    want = rs[:, None] * np.arange(1, N + 1, dtype=np.float64)[None, :]
    bad, err, _ = refs.close(to_np(Zs), want.astype(np.float32))
    assert bad == 0, err


@pytest.mark.parametrize("M,N,K,mode,tm,acc", [(50, 1600, 720, 0, 0, 0), (200, 720, 960, 1, 0, 0), (241, 960, 960, 0, 0, 0),
                                               (50, 720, 2048, 2, 25, 1), (200, 4096, 720, 0, 0, 0)])
def test_xmcast_small_m_shapes(lib, gpu, M, N, K, mode, tm, acc):
    """sh_gemm_xmcast_ex on the small-M GEMM shapes of docs/XPANEL_MCAST.md section 3 (SmolVLA expert and prefix),
    every schedule mode, rows-per-block and accumulate; integer-valued data as the reference's run (exact), and
    normal data against the fp32 product."""
    import torch
    for fill in ("int", "normal"):
        if fill == "int":
            x, w = lcg.fill_fp16(M, K, 81, -2, 2), lcg.fill_fp16(K, N, 82, -2, 2)
        else:
            x, w = data.normal((M, K), 83), data.normal((K, N), 84, std=1 / np.sqrt(K))
        z0 = lcg.fill_fp16(M, N, 85, -3, 3)
        X, W, Z = to_dev(x), to_dev(w), to_dev(z0)
        rc = lib.sh_gemm_xmcast_ex(A(X), A(W), A(Z), M, N, K, K, N, N, shops.cfg(tm, 0, 0, accumulate=acc), mode)
        assert rc == 0, shops.last_error()
        # accumulate stores r16(z0 + r16(X W)) (the product is rounded where sh_gemm would store it)
        want = refs.r16(refs.gemm(x, w)) + z0.astype(np.float32) if acc else refs.gemm(x, w)
        got = to_np(Z)
        if fill == "int":
            assert np.array_equal(got.astype(np.float32), refs.r16(want))
        else:
            bad, err, _ = refs.close(got, want)
            assert bad == 0, err


@pytest.mark.parametrize("K", [8, 40, 136, 720])
@pytest.mark.parametrize("splits", [1, 3])
def test_k_tail_on_direct_to_lds_tiles(lib, gpu, monkeypatch, K, splits):
    """K % 64 != 0 with vector operands (K % 8 == 0) on the direct-to-LDS k_gemm2 tiles: the last, partial 64-k
    slice reads zeros past K, so every k_gemm2 tile (128x128 to 256x256, 64x64 to 128x64; 2 or 3 stages) stores
    the same bits, within tolerance of the oracle, with a bias + GELU epilogue, and nothing outside the view
    changes. K = 8 is a single partial slice; K = 720 is the SmolVLA width (11 slices + 16)."""
    import torch
    M, N, ldz = 200, 328, 336
    x, w = data.normal((M, K), 91), data.normal((K, N), 92, std=1 / np.sqrt(K))
    b = data.normal((1, N), 93, std=0.3).astype(np.float16)
    X, W, Bb = to_dev(x), to_dev(w), to_dev(b)
    outs = {}
    for cfg_index in K2_CFGS:
        monkeypatch.setenv("SH_GEMM_CFG", str(cfg_index))
        Z = torch.full((M + 2, ldz), 7.0, dtype=torch.float16, device="cuda")
        e = shops.epi(bias=A(Bb), act=shops.SH_ACT_GELU, splits=splits)
        assert lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, ldz, None, e) == 0, shops.last_error()
        z = to_np(Z)
        assert (z[:M, N:] == 7.0).all() and (z[M:] == 7.0).all(), cfg_index
        outs[cfg_index] = z[:M, :N].copy()
    ref = outs[K2_CFGS[0]]
    for i, z in outs.items():
        assert np.array_equal(z.view(np.uint16), ref.view(np.uint16)), f"config {i} differs from config {K2_CFGS[0]}"
    want = refs.gelu(refs.r16(refs.r16(refs.gemm(x, w)) + b.astype(np.float32)))
    bad, err, _ = refs.close(ref, want)
    assert bad == 0, err
