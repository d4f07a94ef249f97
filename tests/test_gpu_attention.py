"""Fused attention on the GPU: the reference's logged device outputs (tests/golden), the oracle on the
BASELINE config-4 shapes (B=32 S=256 and B=8 S=1024, 12 heads of 64), QKV-buffer views (ld = 2304,
attention_translate.mlir:23-25), ragged S, other head widths, element-wise paths and scale edge cases."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import lcg, refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
A = shops.addr
ALL = shops.SH_ALL
GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_s256_d768_h12.json"


def _zeros(rows, cols):
    import torch
    return torch.zeros((rows, cols), dtype=torch.float16, device="cuda")


def test_reference_log_through_the_library(lib, gpu):
    """attention/main.c end to end on the GPU: inputs filled by sh_test_fill_fp16 (seeds 21/22/23), output
    poisoned with 7.0 (seed 24), sh_attention_q(..., SH_ALL, 0), then the O0 / O sample dumps."""
    S, D, H = 256, 768, 12
    q, k, v, o = _zeros(S, D), _zeros(S, D), _zeros(S, D), _zeros(S, D)
    lib.sh_test_fill_fp16(A(q), S, D, D, 21, -8, 8, 0.125)
    lib.sh_test_fill_fp16(A(k), S, D, D, 22, -8, 8, 0.125)
    lib.sh_test_fill_fp16(A(v), S, D, D, 23, -16, 16, 0.125)
    lib.sh_test_fill_fp16(A(o), S, D, D, 24, 7, 7, 1.0)
    assert lib.sh_attention_q(A(q), A(k), A(v), A(o), S, D, H, D, D, D, D, 0.125, ALL, 0) == 0, shops.last_error()
    with shops.capture() as cap:
        lib.sh_test_dump_samples(A(o), S, D // H, D, 301, 256, b"O0")
        lib.sh_test_dump_samples(A(o), S, D, D, 302, 256, b"O")
    got = lcg.parse_samples(cap.text)
    fx = json.loads(GOLDEN.read_text())
    ref = refs.attention_reference_lcg(S, D, H)
    for tag, arr in (("O0", ref[:, :64]), ("O", ref)):
        logged = [(r, c, float(np.array([int(h, 16)], np.uint16).view(np.float16)[0])) for r, c, h in fx["samples"][tag]]
        assert [(r, c) for r, c, _ in got[tag]] == [(r, c) for r, c, _ in logged]
        dev_ref = np.zeros_like(arr)
        for r, c, val in logged:
            dev_ref[r, c] = val
        assert lcg.compare_samples(got[tag], dev_ref, 0.05, 0.05)[0] == 0      # vs the reference device, its tolerance
        assert lcg.compare_samples(got[tag], arr, 2e-2, 1e-2)[0] == 0          # vs the oracle
    bad, err, _ = refs.close(to_np(o), ref)
    assert bad == 0, err


def test_qkv_views_and_q_block(lib, gpu):
    """q/k/v as column views of one [256 x 2304] QKV buffer (ld 2304), o with ld 768; q_block 64 and 0."""
    S, D, H = 256, 768, 12
    qkv = data.normal((S, 3 * D), 1)
    QKV = to_dev(qkv)
    for sq in (64, 0):
        O = _zeros(S, D)
        rc = lib.sh_attention_q(A(QKV), A(QKV, D), A(QKV, 2 * D), A(O), S, D, H, 3 * D, 3 * D, 3 * D, D, 0.125, ALL, sq)
        assert rc == 0
        want = refs.attention(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], H, 0.125)
        bad, err, _ = refs.close(to_np(O), want)
        assert bad == 0, err
    O = _zeros(S, 64)
    assert lib.sh_attention_head(A(QKV, 64), A(QKV, D + 64), A(QKV, 2 * D + 64), A(O), S, 64, 3 * D, 3 * D, 3 * D, 64, 0.125, 3) == 0
    want = refs.attention(qkv[:, 64:128], qkv[:, D + 64:D + 128], qkv[:, 2 * D + 64:2 * D + 128], 1, 0.125)
    assert refs.close(to_np(O), want)[0] == 0


@pytest.mark.parametrize("B,S", [(32, 256), (8, 1024)])
def test_baseline_config4_batched(lib, gpu, B, S):
    D, H = 768, 12
    q, k, v = data.normal((B * S, D), 11), data.normal((B * S, D), 12), data.normal((B * S, D), 13)
    O = _zeros(B * S, D)
    rc = lib.sh_attention_batched(A(to_dev(q)), A(to_dev(k)), A(to_dev(v)), A(O), B, S, D, H, D, D, D, D,
                                  S * D, S * D, S * D, S * D, 0.125, 64)
    assert rc == 0, shops.last_error()
    want = refs.attention_batched(q, k, v, B, H, 0.125)
    bad, err, _ = refs.close(to_np(O), want)
    assert bad == 0, err


@pytest.mark.parametrize("S,D,H", [(100, 128, 2), (260, 384, 6), (36, 96, 3), (512, 1536, 12), (64, 576, 12), (20, 72, 2),
                                   (12, 128, 2), (40, 256, 2), (1, 768, 12), (130, 1536, 12)])
def test_shapes_ragged_and_head_widths(lib, gpu, S, D, H):
    """Ragged S (masked last key block), dh = 64 / 32 / 128 / 48 (padded) / 36 (element-wise path)."""
    q, k, v = data.normal((S, D), S), data.normal((S, D), S + 1), data.normal((S, D), S + 2)
    O = _zeros(S, D)
    rc = lib.sh_attention_batched(A(to_dev(q)), A(to_dev(k)), A(to_dev(v)), A(O), 1, S, D, H, D, D, D, D, 0, 0, 0, 0, 0.125, 0)
    assert rc == 0, shops.last_error()
    bad, err, _ = refs.close(to_np(O), refs.attention(q, k, v, H, 0.125))
    assert bad == 0, err


def test_wide_heads_row_kernel(lib, gpu):
    S, D, H = 96, 512, 2            # dh = 256 > 128: per-query kernel
    q, k, v = data.normal((S, D), 5), data.normal((S, D), 6), data.normal((S, D), 7)
    O = _zeros(S, D)
    assert lib.sh_attention(A(to_dev(q)), A(to_dev(k)), A(to_dev(v)), A(O), S, D, H, D, D, D, D, 1 / 16, ALL) == 0
    bad, err, _ = refs.close(to_np(O), refs.attention(q, k, v, H, 1 / 16))
    assert bad == 0, err


@pytest.mark.parametrize("scale", [-0.125, 0.0, 0.6, 1.0])
def test_scale_edge_cases(lib, gpu, scale):
    """Scales whose c = scale log2(e) folds into the query fragments (|c| <= 1: the one-pass kernel) and one that does
    not (1.0: the two-pass kernel without the fold)."""
    S, D, H = 192, 256, 4
    q, k, v = data.normal((S, D), 8), data.normal((S, D), 9), data.normal((S, D), 10)
    O = _zeros(S, D)
    assert lib.sh_attention(A(to_dev(q)), A(to_dev(k)), A(to_dev(v)), A(O), S, D, H, D, D, D, D, scale, ALL) == 0
    bad, err, _ = refs.close(to_np(O), refs.attention(q, k, v, H, scale))
    assert bad == 0, err


@pytest.mark.parametrize("first", [-30.0, -200.0])
@pytest.mark.parametrize("S", [256, 230])
def test_running_reference_moves(lib, gpu, S, first):
    """Scores laid out so the one-pass kernel's reference m moves in every way it can: the first key block's scaled
    scores sit near `first` (m moves down from 0; at -200, 2^200 would overflow fp32 if the still-empty O and l were
    rescaled), the second near -10 and the third near +5 (m moves up by more than 8 after the first block), the last
    near 0 (no move; with S = 230 a partial block). Every query sees the same score pattern (q rows of ones), the keys
    add a little noise, V is random."""
    dh, scale = 64, 0.125
    c = scale * np.log2(np.e)
    rng = np.random.default_rng(7)
    level = np.select([np.arange(S) < 64, np.arange(S) < 128, np.arange(S) < 192], [first, -10.0, 5.0], 0.0)
    q = np.ones((S, dh), np.float32)
    k = (level[:, None] / (c * dh) + 0.05 * rng.standard_normal((S, dh))).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((S, dh)).astype(np.float16).astype(np.float32)
    O = _zeros(S, dh)
    assert lib.sh_attention_batched(A(to_dev(q)), A(to_dev(k)), A(to_dev(v)), A(O), 1, S, dh, 1, dh, dh, dh, dh,
                                    0, 0, 0, 0, scale, 0) == 0, shops.last_error()
    o = to_np(O)
    assert np.isfinite(o).all()
    bad, err, _ = refs.close(o, refs.attention(q, k, v, 1, scale))
    assert bad == 0, err


def test_profile_reports_the_kernel_time(lib, gpu):
    S, D, H = 256, 768, 12
    q = to_dev(data.normal((S, D), 1))
    O = _zeros(S, D)
    assert lib.sh_attention(A(q), A(q), A(q), A(O), S, D, H, D, D, D, D, 0.125, ALL) == 0
    lib.sh_barrier_global()
    assert lib.sh_attention_profile(S, 64, 6) > lib.sh_attention_profile(S, 64, 7) == 0


@pytest.mark.parametrize("S", [256, 1024])
def test_profile_phase_stamps_are_monotone(lib, gpu, S):
    """sh_attention_profile (reference sh_attention.inc.c:67-76, sh_ops.h:124-127): the last workgroup's stamps in
    ns from the first workgroup's start (phase 7 = 0): start (0) <= operands staged (1, 2) <= first key block's
    scores (3, 4) <= every key block done (5) <= stored (6). A batched call leaves
    no stamps (every phase reads 0)."""
    D, H = 768, 12
    q = to_dev(data.normal((S, D), 3))
    O = _zeros(S, D)
    assert lib.sh_attention(A(q), A(q), A(q), A(O), S, D, H, D, D, D, D, 0.125, ALL) == 0
    lib.sh_barrier_global()
    ph = [lib.sh_attention_profile(S, 64, p) for p in range(8)]
    assert ph[7] == 0
    assert ph[0] <= ph[1] <= ph[2] <= ph[3] <= ph[4] <= ph[5] <= ph[6], ph
    assert 0 < ph[6] < 10_000_000 and ph[6] > ph[0], ph
    assert lib.sh_attention_batched(A(q), A(q), A(q), A(O), 1, S, D, H, D, D, D, D, 0, 0, 0, 0, 0.125, 0) == 0
    lib.sh_barrier_global()
    assert all(lib.sh_attention_profile(S, 64, p) == 0 for p in range(8))


@pytest.mark.parametrize("S,dh", [(256, 64), (320, 64), (1024, 128)])
def test_stamped_call_stores_the_bits_of_the_batched_call(lib, gpu, S, dh):
    """sh_attention (a stamped launch: the build that writes the phase stamps) and sh_attention_batched with B=1 (the
    build without any stamp code) store the same bits, ragged last key block included."""
    import torch
    H = 768 // dh
    D = H * dh
    q, k, v = (to_dev(data.normal((S, D), 60 + i)) for i in range(3))
    O1, O2 = _zeros(S, D), _zeros(S, D)
    sc = 1 / dh ** 0.5
    assert lib.sh_attention(A(q), A(k), A(v), A(O1), S, D, H, D, D, D, D, sc, ALL) == 0, shops.last_error()
    lib.sh_barrier_global()
    assert lib.sh_attention_profile(S, dh, 6) > 0
    assert lib.sh_attention_batched(A(q), A(k), A(v), A(O2), 1, S, D, H, D, D, D, D, 0, 0, 0, 0, sc, 0) == 0
    torch.cuda.synchronize()
    assert torch.equal(O1.view(torch.int16), O2.view(torch.int16))


@pytest.mark.parametrize("dh,scale", [(64, 0.125), (128, 0.088), (64, 1.0)])
def test_batched_prefetch_stores_the_bits_of_batched(lib, gpu, dh, scale):
    """sh_attention_batched_prefetch with two ranges (unaligned ends, one of them larger than the lines the one-pass
    kernel's threads cover in one pass) stores the bits of sh_attention_batched and leaves the ranges unchanged;
    scale 1.0 does not fold into the queries, so the two-pass kernel runs and the ranges are read after it."""
    import torch
    B, S, H = 3, 320, 4
    D = H * dh
    q, k, v = (to_dev(data.normal((B * S, D), 40 + i)) for i in range(3))
    O1, O2 = _zeros(B * S, D), _zeros(B * S, D)
    g = torch.Generator(device="cuda").manual_seed(4)
    r0 = torch.randint(-30000, 30000, (6 << 20,), dtype=torch.int16, device="cuda", generator=g)
    r1 = torch.randint(-30000, 30000, (3 << 20,), dtype=torch.int16, device="cuda", generator=g)
    keep = (r0.clone(), r1.clone())
    args = (A(q), A(k), A(v), None, B, S, D, H, D, D, D, D, S * D, S * D, S * D, S * D, scale, 0)
    assert lib.sh_attention_batched(*args[:3], A(O1), *args[4:]) == 0, shops.last_error()
    assert lib.sh_attention_batched_prefetch(*args[:3], A(O2), *args[4:], A(r0) + 6, (12 << 20) - 20,
                                             A(r1) + 130, 1000) == 0, shops.last_error()
    torch.cuda.synchronize()
    assert torch.equal(O1.view(torch.int16), O2.view(torch.int16))
    assert torch.equal(r0, keep[0]) and torch.equal(r1, keep[1])
    assert lib.sh_attention_batched_prefetch(*args[:3], A(O2), *args[4:], 0, 64, 0, 0) == -1      # NULL range
