"""Test helpers of the library on the GPU (reference runtime/sh_test.inc.c): the LCG fills are bit-identical
to the oracle's sequential generator (including across the jump-ahead boundaries of the GPU kernel), the
sample dump follows the "<tag> r c hex" protocol, constant fills/checks, the runtime's timers and arena."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import codes, to_np
from oracle import lcg
from softhier_mlir_amd import shops

pytestmark = pytest.mark.gpu
A = shops.addr


def _buf(rows, cols, fill=0.0):
    import torch
    return torch.full((rows, cols), fill, dtype=torch.float16, device="cuda")


@pytest.mark.parametrize("rows,cols,seed,lo,hi,scale", [(256, 768, 1, -16, 16, 0.125), (3, 5, 7, -1, 1, 1.0),
                                                        (768, 3072, 6, -8, 8, 1 / 128), (4096, 1800, 23, -16, 16, 0.125)])
def test_fill_is_bit_identical_to_the_sequential_lcg(lib, gpu, rows, cols, seed, lo, hi, scale):
    B = _buf(rows, cols + 8, 7.0)                       # ld = cols + 8: the padding keeps its poison
    lib.sh_test_fill_fp16(A(B), rows, cols, cols + 8, seed, lo, hi, scale)
    got = codes(B)
    assert np.array_equal(got[:, :cols], lcg.fill_fp16(rows, cols, seed, lo, hi, scale).view(np.uint16))
    assert (got[:, cols:] == np.float16(7.0).view(np.uint16)).all()


def test_dump_protocol_and_idx(lib, gpu):
    B = _buf(64, 96)
    lib.sh_test_fill_int_fp16(A(B), 64, 96, 96, 5, -4, 4)
    with shops.capture() as cap:
        lib.sh_test_dump_samples(A(B), 64, 96, 96, 9, 32, b"P")
        lib.sh_test_dump_samples_idx(A(B), 64, 96, 96, 9, 4, b"L", 3)
    s = lcg.parse_samples(cap.text)
    ref = lcg.fill_fp16(64, 96, 5, -4, 4)
    assert [(r, c) for r, c, _ in s["P"]] == lcg.sample_positions(64, 96, 9, 32)
    assert all(ref[r, c] == v for r, c, v in s["P"])
    assert len(s["L3"]) == 4
    with shops.capture() as cap:
        lib.sh_test_dump_all(A(B), 2, 3, 96, b"Z")
    assert cap.text.splitlines()[0] == f"Z 0 0 {int(ref[0, 0:1].view(np.uint16)[0]):04x}"


def test_const_fills_and_checks(lib, gpu):
    B = _buf(16, 40)
    lib.sh_test_fill_const_fp16(A(B), 16, 40, 40, 0x3C00)
    with shops.capture() as cap:
        ok = lib.sh_test_check_const_fp16(A(B), 16, 40, 40, 0x3C00, 0, b"C")
    assert ok == 640 and "C_CHECK ok=640/640 C_PASS" in cap.text
    lib.sh_test_fill_colparity_fp16(A(B), 16, 40, 40, 0x3C00, 0x3800)
    assert np.array_equal(codes(B), lcg.col_parity_fp16(16, 40, 0x3C00, 0x3800).view(np.uint16))
    with shops.capture() as cap:
        ok = lib.sh_test_check_const_fp16(A(B), 16, 40, 40, 0x3C00, 0, b"C")
    assert ok == 320 and "C_FAIL" in cap.text


def test_timer_arena_and_cycles(lib, gpu):
    with shops.capture() as cap:
        lib.sh_timer_start()
        B = _buf(1024, 1024)
        lib.sh_test_fill_fp16(A(B), 1024, 1024, 1024, 1, -1, 1, 1.0)
        lib.sh_timer_end()
    assert cap.text.startswith("[Performance Counter]: Execution period is ") and lib.sh_timer_last_ns() > 0
    a0, a1 = lib.sh_hbm_addr(0x1000), lib.sh_hbm_addr(0x2000)
    assert a0 != 0 and a1 - a0 == 0x1000
    m = lib.sh_hbm_malloc(4096)
    assert m != 0 and m % 256 == 0
    c0 = lib.sh_cycles()
    c1 = lib.sh_cycles()
    assert (c1 - c0) % 2 ** 32 < 10 ** 9


def test_prefetch_reads_ranges_and_writes_nothing(lib, gpu):
    """sh_prefetch on ranges that start and end inside 64-byte lines (and a whole buffer) returns 0 and leaves every
    byte as it was; an empty range does nothing."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(3)
    t = torch.randint(-30000, 30000, (1 << 20,), dtype=torch.int16, device="cuda", generator=g)
    before = t.clone()
    for off, n in ((0, 2 << 20), (6, 1000), (130, 64 * 1001 + 5), ((1 << 20) - 7, 14)):
        assert lib.sh_prefetch(A(t) + off, n) == 0, shops.last_error()
    assert lib.sh_prefetch(A(t), 0) == 0
    torch.cuda.synchronize()
    assert torch.equal(t, before)
