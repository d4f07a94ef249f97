"""Row ops on the GPU against the oracle: the reference's rowops test (run.py:136-173 inputs and formulas,
rowops/main.c op arguments), BASELINE config-3 shapes, strided views, the element-wise paths, rows wider than
the register-resident kernels, in-place calls, and bit-exact transposes (NaN payloads included)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import codes, to_dev, to_np
from oracle import lcg, refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
A = shops.addr
ALL = shops.SH_ALL


def _empty(rows, cols, fill=7.0):
    import torch
    return torch.full((rows, cols), fill, dtype=torch.float16, device="cuda")


@pytest.mark.parametrize("rows,cols", [(64, 96), (256, 768), (33, 40)])
def test_reference_rowops(lib, gpu, rows, cols):
    """run.py run_rowops: LN eps 1e-5, softmax 0.5, gelu, add, add_bias (be row), scale 0.3, transpose."""
    x = lcg.fill_fp16(rows, cols, 11, -16, 16, 0.125)
    b = lcg.fill_fp16(rows, cols, 12, -16, 16, 0.125)
    g = lcg.fill_fp16(1, cols, 13, 1, 8, 0.25)
    be = lcg.fill_fp16(1, cols, 14, -4, 4, 0.25)
    X, Bt, G, BE = to_dev(x), to_dev(b), to_dev(g), to_dev(be)
    out = {k: _empty(rows, cols) for k in ("LN", "SM", "GELU", "ADD", "BIAS", "SCALE")}
    T = _empty(cols, rows)
    lib.sh_layernorm(A(out["LN"]), A(X), A(G), A(BE), rows, cols, cols, 1e-5, ALL)
    lib.sh_softmax_rows(A(out["SM"]), A(X), rows, cols, cols, 0.5, ALL)
    lib.sh_gelu(A(out["GELU"]), A(X), rows, cols, cols, ALL)
    lib.sh_add(A(out["ADD"]), A(X), A(Bt), rows, cols, cols, ALL)
    lib.sh_add_bias(A(out["BIAS"]), A(X), A(BE), rows, cols, cols, ALL)
    lib.sh_scale(A(out["SCALE"]), A(X), rows, cols, cols, 0.3, ALL)
    lib.sh_transpose(A(T), A(X), rows, cols, cols, rows, ALL)
    want = {"LN": refs.layernorm(x, g, be, 1e-5), "SM": refs.softmax(x, 0.5), "GELU": refs.gelu(x),
            "ADD": refs.add(x, b), "BIAS": refs.add_bias(x, be), "SCALE": refs.scale(x, 0.3)}
    for k, w in want.items():
        bad, err, _ = refs.close(to_np(out[k]), w)
        assert bad == 0, (k, err)
    assert np.array_equal(codes(T), refs.transpose(x.view(np.uint16)))
    # the reference's sampled-dump comparison at its own tolerance (run.py:168)
    with shops.capture() as cap:
        lib.sh_test_dump_samples(A(out["LN"]), rows, cols, cols, 101, 64, b"LN")
    s = lcg.parse_samples(cap.text)["LN"]
    assert [(r, c) for r, c, _ in s] == lcg.sample_positions(rows, cols, 101, 64)
    assert lcg.compare_samples(s, want["LN"], 2e-2, 2e-2)[0] == 0


def test_baseline_config3(lib, gpu):
    # layernorm [256 x 768], eps 1e-6, gamma ~ N(1, .02), beta ~ N(0, .02)
    x = data.normal((256, 768), 1)
    g, be = data.normal((1, 768), 2, 1.0, 0.02), data.normal((1, 768), 3, 0.0, 0.02)
    Y = _empty(256, 768)
    lib.sh_layernorm(A(Y), A(to_dev(x)), A(to_dev(g)), A(to_dev(be)), 256, 768, 768, 1e-6, ALL)
    assert refs.close(to_np(Y), refs.layernorm(x, g, be, 1e-6))[0] == 0
    # softmax over the last dim of [12 x 256 x 256], scale 1/8, x ~ N(0, 3)
    s = data.normal((12 * 256, 256), 4, 0.0, 3.0)
    Y = _empty(12 * 256, 256)
    lib.sh_softmax_rows(A(Y), A(to_dev(s)), 12 * 256, 256, 256, 0.125, ALL)
    assert refs.close(to_np(Y), refs.softmax(s, 0.125))[0] == 0
    # tanh-GELU [256 x 3072]
    f = data.normal((256, 3072), 5)
    Y = _empty(256, 3072)
    lib.sh_gelu(A(Y), A(to_dev(f)), 256, 3072, 3072, ALL)
    assert refs.close(to_np(Y), refs.gelu(f))[0] == 0
    # residual add and add_bias [256 x 768]
    a, b, bias = data.normal((256, 768), 6), data.normal((256, 768), 7), data.normal((1, 768), 8)
    Y = _empty(256, 768)
    lib.sh_add(A(Y), A(to_dev(a)), A(to_dev(b)), 256, 768, 768, ALL)
    assert refs.close(to_np(Y), refs.add(a, b))[0] == 0
    lib.sh_add_bias(A(Y), A(to_dev(a)), A(to_dev(bias)), 256, 768, 768, ALL)
    assert refs.close(to_np(Y), refs.add_bias(a, bias))[0] == 0
    # transpose [768 x 256] taken from a strided view (a 768 x 256 block at column 128 of a 768 x 1024 buffer)
    big = data.normal((768, 1024), 9)
    Big = to_dev(big)
    T = _empty(256, 800)                          # ld_dst = 800 > 768
    lib.sh_transpose(A(T), A(Big, 128), 768, 256, 1024, 800, ALL)
    t = codes(T)
    assert np.array_equal(t[:, :768], big[:, 128:384].view(np.uint16).T)
    assert (t[:, 768:] == np.float16(7.0).view(np.uint16)).all()


def test_strided_views_and_in_place(lib, gpu):
    """ld > cols on a 64-column head slice (loop_translate.mlir:33), and y == x (softmax in place, gemm_seq)."""
    x = data.normal((256, 768), 11)
    X = to_dev(x)
    lib.sh_gelu(A(X, 128), A(X, 128), 256, 64, 768, ALL)
    got = to_np(X)
    assert refs.close(got[:, 128:192], refs.gelu(x[:, 128:192]))[0] == 0
    assert np.array_equal(np.delete(got, np.s_[128:192], 1).view(np.uint16), np.delete(x, np.s_[128:192], 1).view(np.uint16))
    s = data.normal((300, 256), 12, 0.0, 3.0)
    S = to_dev(s)
    lib.sh_softmax_rows(A(S), A(S), 300, 256, 256, 0.125, ALL)
    assert refs.close(to_np(S), refs.softmax(s, 0.125))[0] == 0
    n = data.normal((50, 768), 13)
    N = to_dev(n)
    g, be = data.normal((1, 768), 14, 1.0, 0.1), data.normal((1, 768), 15, 0.0, 0.1)
    lib.sh_layernorm(A(N), A(N), A(to_dev(g)), A(to_dev(be)), 50, 768, 768, 1e-6, ALL)
    assert refs.close(to_np(N), refs.layernorm(n, g, be, 1e-6))[0] == 0


@pytest.mark.parametrize("cols", [77, 5, 520, 1100, 8192, 10000])
def test_widths_and_elementwise_paths(lib, gpu, cols):
    """cols % 8 != 0 (element-wise path), register-resident widths up to 8192, wider rows (loop kernel)."""
    rows = 37
    x = data.normal((rows, cols), cols, 0.0, 2.0)
    g, be = data.normal((1, cols), 1, 1.0, 0.1), data.normal((1, cols), 2, 0.0, 0.1)
    b = data.normal((rows, cols), 3)
    X, G, BE, Bt = to_dev(x), to_dev(g), to_dev(be), to_dev(b)
    Y = _empty(rows, cols)
    lib.sh_layernorm(A(Y), A(X), A(G), A(BE), rows, cols, cols, 1e-6, ALL)
    assert refs.close(to_np(Y), refs.layernorm(x, g, be, 1e-6))[0] == 0
    lib.sh_softmax_rows(A(Y), A(X), rows, cols, cols, -0.7, ALL)
    assert refs.close(to_np(Y), refs.softmax(x, -0.7))[0] == 0
    lib.sh_add(A(Y), A(X), A(Bt), rows, cols, cols, ALL)
    assert refs.close(to_np(Y), refs.add(x, b))[0] == 0
    lib.sh_add_bias(A(Y), A(X), A(BE), rows, cols, cols, ALL)
    assert refs.close(to_np(Y), refs.add_bias(x, be))[0] == 0
    lib.sh_scale(A(Y), A(X), rows, cols, cols, -1.75, ALL)
    assert refs.close(to_np(Y), refs.scale(x, -1.75))[0] == 0
    lib.sh_gelu(A(Y), A(X), rows, cols, cols, ALL)
    assert refs.close(to_np(Y), refs.gelu(x))[0] == 0


def test_unaligned_base(lib, gpu):
    """Views starting one element into the buffer (no 16-byte alignment) take the element-wise path."""
    x = data.normal((20, 97), 21)
    X = to_dev(x)
    Y = _empty(20, 97)
    g, be = np.ones((1, 97), np.float16), np.zeros((1, 97), np.float16)
    G, BE = to_dev(g), to_dev(be)
    lib.sh_layernorm(A(Y, 1), A(X, 1), A(G, 1), A(BE, 1), 20, 96, 97, 1e-6, ALL)
    assert refs.close(to_np(Y)[:, 1:], refs.layernorm(x[:, 1:], g[:, 1:], be[:, 1:], 1e-6))[0] == 0
    lib.sh_scale(A(Y, 1), A(X, 1), 20, 96, 97, 2.0, ALL)
    assert refs.close(to_np(Y)[:, 1:], refs.scale(x[:, 1:], 2.0))[0] == 0


@pytest.mark.parametrize("rows,cols", [(768, 256), (256, 768), (136, 264), (13, 29), (1, 1), (3000, 8)])
def test_transpose_bit_exact(lib, gpu, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    c = rng.integers(0, 65536, (rows, cols), dtype=np.uint16)
    c[::3, ::5] = 0x7C01 + (np.arange(c[::3, ::5].size).reshape(c[::3, ::5].shape) % 0x3FE).astype(np.uint16)  # NaN payloads
    X = to_dev(c)
    T = _empty(cols, rows)
    lib.sh_transpose(A(T), A(X), rows, cols, cols, rows, ALL)
    assert np.array_equal(codes(T), c.T)


def test_large_rows_batched_hbm_shapes(lib, gpu):
    """The ×32 batched shapes of the measured configuration, checked through exact invariants at full size:
    LN of x and of (a x + b) agree (scale/shift invariance), softmax rows sum to 1, add is exact on integers."""
    rows, cols = 8192, 768
    x = data.normal((rows, cols), 31)
    X = to_dev(x)
    g, be = np.ones((1, cols), np.float16), np.zeros((1, cols), np.float16)
    Y = _empty(rows, cols)
    lib.sh_layernorm(A(Y), A(X), A(to_dev(g)), A(to_dev(be)), rows, cols, cols, 1e-6, ALL)
    y = to_np(Y).astype(np.float32)
    assert np.abs(y.mean(1)).max() < 2e-3 and np.abs(y.var(1) - 1).max() < 5e-3
    sm = data.normal((12 * 256 * 32, 256), 32, 0.0, 3.0)
    SM = to_dev(sm)
    lib.sh_softmax_rows(A(SM), A(SM), sm.shape[0], 256, 256, 0.125, ALL)
    p = to_np(SM).astype(np.float32)
    assert np.abs(p.sum(1) - 1).max() < 2e-2 and (p >= 0).all()
    ints = lcg.fill_fp16(rows, cols, 33, -512, 512)
    I = to_dev(ints)
    lib.sh_add(A(Y), A(I), A(I), rows, cols, cols, ALL)
    assert np.array_equal(to_np(Y), (2 * ints.astype(np.float32)).astype(np.float16))


@pytest.mark.parametrize("rows,cols,inplace", [(8192, 768, False), (10007, 520, True), (9000, 1024, False)])
def test_layernorm_many_rows_against_oracle(lib, gpu, rows, cols, inplace):
    """Row counts large enough for the pipelined LayerNorm (a fixed grid of waves walking the rows with two
    rows of loads in flight), including a ragged last pass and the in-place form, against the oracle."""
    x = data.normal((rows, cols), 41)
    g, be = data.normal((1, cols), 42, 1.0, 0.02), data.normal((1, cols), 43, 0.0, 0.02)
    X = to_dev(x)
    Y = X if inplace else _empty(rows, cols)
    lib.sh_layernorm(A(Y), A(X), A(to_dev(g)), A(to_dev(be)), rows, cols, cols, 1e-6, ALL)
    bad, err, _ = refs.close(to_np(Y), refs.layernorm(x, g, be, 1e-6))
    assert bad == 0, err


@pytest.mark.parametrize("cols", [8, 64, 72, 136, 256])
@pytest.mark.parametrize("scale", [0.125, -0.7])
def test_softmax_short_rows(lib, gpu, cols, scale):
    """Rows of at most 256 columns take the several-rows-per-wavefront kernel (8, 16 or 32 lanes per row):
    ragged row count (not a multiple of the 32..128 rows a wavefront covers), ld > cols, the padding columns
    of each row left untouched, and the same rows in place."""
    rows, ld = 1001, cols + 24
    x = data.normal((rows, ld), 40 + cols, 0.0, 3.0)
    X = to_dev(x)
    Y = _empty(rows, ld)
    lib.sh_softmax_rows(A(Y), A(X), rows, cols, ld, scale, ALL)
    y = to_np(Y)
    assert refs.close(y[:, :cols], refs.softmax(x[:, :cols], scale))[0] == 0
    assert (y[:, cols:] == 7.0).all()
    lib.sh_softmax_rows(A(X), A(X), rows, cols, ld, scale, ALL)
    xi = to_np(X)
    assert (xi[:, :cols].view(np.uint16) == y[:, :cols].view(np.uint16)).all()
    assert (xi[:, cols:].view(np.uint16) == x[:, cols:].view(np.uint16)).all()


@pytest.mark.parametrize("nbytes,so,do", [(16 << 20, 0, 0), (4096 + 48, 16, 32), (1000003, 3, 5), (1, 0, 7),
                                         ((160 << 20) + 48, 16, 32), ((256 << 20) + 48, 16, 32)])
def test_dma_copy_moves_every_byte(lib, gpu, nbytes, so, do):
    """sh_dma_copy (sh_ops.h:218): a 1-D copy of exactly `bytes`, aligned (streaming 16-byte path; from 128 MiB one
    chunk per thread with nontemporal stores) or not (byte path), leaving the bytes around the destination range
    untouched."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(5)
    src = torch.randint(0, 256, (nbytes + so + 64,), dtype=torch.uint8, device="cuda", generator=g)
    dst = torch.full((nbytes + do + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    lib.sh_dma_copy(shops.addr(dst, do), shops.addr(src, so), nbytes)
    torch.cuda.synchronize()
    assert torch.equal(dst[do:do + nbytes], src[so:so + nbytes])
    assert (dst[:do] == 0xA5).all() and (dst[do + nbytes:] == 0xA5).all()


def test_elementwise_above_the_infinity_cache(lib, gpu):
    """Outputs of 128 MiB and more take the one-item-per-thread launch with nontemporal stores: on a [131072 x 1024]
    tensor tiled from one 64-row block, every block of the GELU, add_bias and scale outputs equals the library's
    result on the block alone (bit for bit: the same element-wise function), and add of integers is exact."""
    import torch
    rows, cols, blk = 131072, 1024, 64
    x = data.normal((blk, cols), 41, 0.0, 2.0)
    be = data.normal((1, cols), 42, 0.0, 0.1)
    Xs, BE = to_dev(x), to_dev(be)
    Xb = Xs.repeat(rows // blk, 1)
    Ys, Yb = _empty(blk, cols), _empty(rows, cols)
    for name, call in (("gelu", lambda y, x_, r: lib.sh_gelu(A(y), A(x_), r, cols, cols, ALL)),
                       ("add_bias", lambda y, x_, r: lib.sh_add_bias(A(y), A(x_), A(BE), r, cols, cols, ALL)),
                       ("scale", lambda y, x_, r: lib.sh_scale(A(y), A(x_), r, cols, cols, -1.75, ALL))):
        call(Ys, Xs, blk)
        call(Yb, Xb, rows)
        torch.cuda.synchronize()
        want = Ys.view(torch.int16).repeat(rows // blk, 1)
        assert torch.equal(Yb.view(torch.int16), want), name
    assert refs.close(to_np(Ys), refs.scale(x, -1.75))[0] == 0
    ints = to_dev(lcg.fill_fp16(blk, cols, 43, -512, 512)).repeat(rows // blk, 1)
    lib.sh_add(A(Yb), A(ints), A(ints), rows, cols, cols, ALL)
    torch.cuda.synchronize()
    assert torch.equal(Yb, ints * 2)



def test_row_ops_above_the_infinity_cache(lib, gpu):
    """LayerNorm, softmax and transpose on tensors of 128 MiB and more take their nontemporal builds (nontemporal
    stores; softmax and transpose also nontemporal loads; LayerNorm walks rows over at most 32 blocks per CU): on
    inputs tiled from one 64-row block, every block of the output equals the library's result on the block alone,
    bit for bit (each row is reduced by one lane group in the same order), and that result matches the oracle."""
    import torch
    blk = 64
    for name, rows, cols in (("layernorm", 131072, 768), ("softmax", 262144, 256), ("transpose", 131072, 768)):
        x = data.normal((blk, cols), 44, 0.5, 1.5)
        Xs = to_dev(x)
        Xb = Xs.repeat(rows // blk, 1)
        if name == "layernorm":
            g, be = data.normal((1, cols), 45, 1.0, 0.2), data.normal((1, cols), 46, 0.0, 0.2)
            G, BE = to_dev(g), to_dev(be)
            Ys, Yb = _empty(blk, cols), _empty(rows, cols)
            lib.sh_layernorm(A(Ys), A(Xs), A(G), A(BE), blk, cols, cols, 1e-5, ALL)
            lib.sh_layernorm(A(Yb), A(Xb), A(G), A(BE), rows, cols, cols, 1e-5, ALL)
            want = refs.layernorm(x, g, be, 1e-5)
        elif name == "softmax":
            Ys, Yb = _empty(blk, cols), _empty(rows, cols)
            lib.sh_softmax_rows(A(Ys), A(Xs), blk, cols, cols, 0.7, ALL)
            lib.sh_softmax_rows(A(Yb), A(Xb), rows, cols, cols, 0.7, ALL)
            want = refs.softmax(x, 0.7)
        else:
            Ys, Yb = _empty(cols, blk), _empty(cols, rows)
            lib.sh_transpose(A(Ys), A(Xs), blk, cols, cols, blk, ALL)
            lib.sh_transpose(A(Yb), A(Xb), rows, cols, cols, rows, ALL)
        torch.cuda.synchronize()
        assert shops.last_error()[0] == 0, (name, shops.last_error())
        if name == "transpose":
            assert np.array_equal(codes(Ys), codes(Xs).T), name
            assert torch.equal(Yb.view(torch.int16), Ys.view(torch.int16).repeat(1, rows // blk)), name
        else:
            assert torch.equal(Yb.view(torch.int16), Ys.view(torch.int16).repeat(rows // blk, 1)), name
            assert refs.close(to_np(Ys), want)[0] == 0, name
        del Xb, Yb
