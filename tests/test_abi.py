"""The C ABI without a GPU: libshops.so loads, exports every function include/sh_ops.h declares, and its
host-only functions (codec, budgets, q-block rule, argument validation) behave as the reference's."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from softhier_mlir_amd import shops


def test_library_exports_every_header_function(lib):
    names = shops.header_functions()
    assert len(names) >= 55
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    # every bound signature names a header function (no stale bindings)
    assert set(shops._SIGS) | shops._UNTYPED <= set(names)


def test_struct_layouts_match_the_reference():
    assert C.sizeof(shops.sh_gemm_cfg) == 28            # 7 x uint32 (reference runtime/sh_ops.h:54-60)
    assert [f for f, _ in shops.sh_gemm_cfg._fields_] == ["tm", "tn", "tk", "pipeline", "accumulate", "fmt", "l1_base"]
    assert shops.SH_ALL == 0xFFFFFFFF


def test_host_fp16_codec_exhaustive(lib):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([lib.sh_fp16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_host_fp16_encode(lib):
    rng = np.random.default_rng(3)
    u = rng.integers(0, 2 ** 32, 50_000, dtype=np.uint64).astype(np.uint32)
    u[1::2] = (u[1::2] & 0x807FFFFF) | (((u[1::2] >> 8) % 40 + 100) << 23)
    u[3::8] = (u[3::8] & ~np.uint32(0x1FFF)) | np.uint32(0x1000)          # ties at the rounding bit
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    got = np.array([lib.sh_f32_to_fp16(float(v)) for v in f], np.uint16)
    assert np.array_equal(got, want)
    assert lib.sh_f32_to_fp16(float("nan")) == 0x7E00   # canonical quiet NaN (reference sh_rt.inc.c:47)


def test_runtime_identity_functions(lib):
    assert lib.sh_cluster_id() == 0 and lib.sh_core_id() == 0
    assert lib.sh_is_first_core() == 1 and lib.sh_is_dm_core() == 1
    assert lib.sh_num_clusters() == 1
    assert lib.sh_l1_size() == 0x100000


def test_gemm_l1_bytes_formula(lib):
    # sh_gemm.inc.c:24-30: l1_base + (pipeline ? 2 : 1) * (tm tk + tk tn) * 2 + tm tn * 2, defaults 256
    assert lib.sh_gemm_l1_bytes(256, 256, 256, None) == 2 * (2 * 256 * 256 * 2) + 256 * 256 * 2
    c = shops.cfg(256, 256, 64, pipeline=1)
    assert lib.sh_gemm_l1_bytes(256, 256, 64, c) == 2 * (256 * 64 * 2 + 64 * 256 * 2) + 256 * 256 * 2
    c = shops.cfg(128, 64, 32, pipeline=0, l1_base=4096)
    assert lib.sh_gemm_l1_bytes(1, 1, 1, c) == 4096 + (128 * 32 * 2 + 32 * 64 * 2) + 128 * 64 * 2


def test_attention_budget_and_q_block_match_the_reference_log(lib):
    # tests/gvsoc/attention/last_run.log: "l1=300064 B", "q block 64 rows: 48 work items" (S=256, dh=64, H=12, 16 clusters)
    assert lib.sh_attention_l1_bytes(256, 64) == 300064
    assert lib.sh_attention_q_block(256, 64, 12, 16) == 64
    assert lib.sh_attention_q_block(256, 64, 1, 1) == 256
    assert lib.sh_attention_q_block(1024, 64, 12, 16) == 256    # S=1024 fits with sq=256 (961 KB, sh_attention.inc.c:7)
    assert lib.sh_attention_l1_bytes_q(1024, 64, 256) < 0x100000 < lib.sh_attention_l1_bytes_q(1024, 64, 1024)
    assert lib.sh_attention_q_block(4096, 64, 12, 16) == 0      # nothing fits the reference TCDM


def test_gemm_argument_errors_without_gpu(lib):
    one = 1 << 20                                               # never dereferenced: validation fails first
    assert lib.sh_gemm(one, one, one, 100, 256, 256, 256, 256, 256, None, shops.SH_ALL) == -1   # M % 256
    assert shops.last_error()[0] == -1
    c = shops.cfg(512, 512, 512)
    assert lib.sh_gemm(one, one, one, 512, 512, 512, 512, 512, 512, c, 0) == -2                # TCDM budget
    assert shops.last_error()[0] == -2
    c = shops.cfg(256, 128, 256)
    assert lib.sh_gemm_mesh(one, one, one, 1024, 1024, 1024, 1024, 1024, 1024, c) == -1         # tm != tn
    c = shops.cfg(256, 256, 256)
    assert lib.sh_gemm_mesh(one, one, one, 512, 512, 512, 512, 512, 512, c) == -1              # M != 4 tm
    assert lib.sh_gemm(0, one, one, 256, 256, 256, 256, 256, 256, None, 0) == -1                # NULL
    c = shops.cfg(fmt=shops.SH_FP8)
    assert lib.sh_gemm(one, one, one, 256, 256, 256, 256, 256, 256, c, 0) == -1                # fp8 not implemented
    e = shops.epi(residual=one, ldr=10)
    assert lib.sh_gemm_ex(one, one, one, 16, 32, 16, 16, 32, 32, None, e) == -1                 # ldr < N


def test_xmcast_plan_follows_the_reference_schedules(lib):
    """sh_gemm_xmcast_l1_bytes / plan (sh_gemm.inc.c:219-258) against what docs/XPANEL_MCAST.md reports: the column
    slice of N=1600 on 16 clusters is 100 (1600/16 rounded up to the granule 4), K panels are the largest divisor
    of K <= 256 that fits, and AUTO picks the whole-X schedule up to 320 KB of X (50x1600x720, 200x1600x720) and
    panels above it (200x720x960: X = 384 KB; 400x1600x720)."""
    X, P, W = shops.SH_XM_AUTO, shops.SH_XM_PANEL, shops.SH_XM_WHOLE
    # whole X, M=50, N=1600, K=720: X 72000 B + two W panels (tk=240, Nc=100) + Y (50 x 100)
    assert lib.sh_gemm_xmcast_l1_bytes(50, 1600, 720, None, W) == 50 * 720 * 2 + 2 * 240 * 100 * 2 + 50 * 100 * 2
    for m, n, k, whole in ((50, 1600, 720, True), (200, 1600, 720, True), (200, 720, 960, False), (400, 1600, 720, False)):
        auto = lib.sh_gemm_xmcast_l1_bytes(m, n, k, None, X)
        assert auto == lib.sh_gemm_xmcast_l1_bytes(m, n, k, None, W if whole else P) != 0xFFFFFFFF
    # panel schedule of 200x720x960: Nc = ceil(720/16)=45 -> 48; tk = 240 (largest divisor of 960 <= 256)
    assert lib.sh_gemm_xmcast_l1_bytes(200, 720, 960, None, P) == 2 * 200 * 240 * 2 + 2 * 240 * 48 * 2 + 200 * 48 * 2
    # explicit tk must divide K; rows per block must divide M; l1_base at the limit leaves no plan
    assert lib.sh_gemm_xmcast_l1_bytes(50, 1600, 720, shops.cfg(0, 0, 7), P) == 0xFFFFFFFF
    assert lib.sh_gemm_xmcast_l1_bytes(50, 1600, 720, shops.cfg(16, 0, 0), P) == 0xFFFFFFFF
    assert lib.sh_gemm_xmcast_l1_bytes(50, 1600, 720, shops.cfg(l1_base=0x90000), P) == 0xFFFFFFFF
    # whole X of 50 x 8192 x 2 = 800 KB cannot fit: WHOLE has no plan, AUTO falls back to panels
    assert lib.sh_gemm_xmcast_l1_bytes(50, 256, 8192, None, W) == 0xFFFFFFFF
    assert lib.sh_gemm_xmcast_l1_bytes(50, 256, 8192, None, X) == lib.sh_gemm_xmcast_l1_bytes(50, 256, 8192, None, P)


def test_xmcast_argument_errors_without_gpu(lib):
    one = 1 << 20
    assert lib.sh_gemm_xmcast_ex(one, one, one, 50, 64, 64, 64, 64, 64, shops.cfg(16, 0, 0), shops.SH_XM_AUTO) == -1
    assert lib.sh_gemm_xmcast_ex(one, one, one, 50, 64, 64, 64, 64, 64, shops.cfg(l1_base=0x90000), 0) == -2
    assert lib.sh_gemm_xmcast(one, one, one, 50, 64, 64, 64, 64, 64, shops.cfg(fmt=shops.SH_FP8)) == -3
    assert shops.last_error()[0] == -3
    assert lib.sh_gemm_xmcast(0, one, one, 50, 64, 64, 64, 64, 64, None) == -1


def test_attention_argument_errors_without_gpu(lib):
    one = 1 << 20
    assert lib.sh_attention(one, one, one, one, 256, 768, 7, 768, 768, 768, 768, 0.125, shops.SH_ALL) == -1  # D % H
    assert lib.sh_attention_q(one, one, one, one, 256, 768, 12, 768, 768, 768, 768, 0.125, 0, 96) == -1    # sq ∤ S
    assert lib.sh_attention_q(one, one, one, one, 258, 768, 12, 768, 768, 768, 768, 0.125, 0, 0) == -1     # S % 4
    assert lib.sh_attention_head(one, one, one, one, 4096, 64, 64, 64, 64, 64, 0.125, 0) == -1          # budget
    assert lib.sh_attention_batched(one, one, one, one, 2, 256, 768, 5, 768, 768, 768, 768, 0, 0, 0, 0, 0.125, 0) == -1


def test_rowop_argument_errors_without_gpu(lib):
    lib.sh_last_error()
    lib.sh_layernorm(0, 1 << 20, 1 << 20, 1 << 20, 4, 8, 8, 1e-6, 0)
    assert shops.last_error()[0] == -1
    lib.sh_transpose(1 << 20, 1 << 20, 4, 8, 4, 4, 0)           # ld_src < cols
    assert shops.last_error()[0] == -1
    lib.sh_add(1 << 20, 1 << 20, 1 << 20, 0, 8, 8, 0)           # zero rows: nothing to do, no error
    assert shops.last_error()[0] == 0


def test_capture_collects_library_text(lib):
    with shops.capture() as cap:
        lib.sh_printf(b"hello %d\n", C.c_int(7))
    assert cap.text == "hello 7\n"


def test_gemm_tile_plan_without_gpu(lib):
    """The GEMM cost model (sh_gemm_plan, no GPU work): small problems take the small direct-to-LDS tiles
    (latency-bound: many short workgroups), the encoder's M = 8192 shapes the 128 x 192 tiles whose choice the
    one-time timing refines, explicit split requests are kept, and K % 64 != 0 stays on a direct-to-LDS tile."""
    import ctypes as C

    def plan(M, N, K, splits=0):
        out = (C.c_uint32 * 4)()
        assert lib.sh_gemm_plan(M, N, K, splits, out) == 0
        return tuple(out)
    for M, N, K in [(256, 2304, 768), (256, 3072, 768), (256, 256, 256), (1024, 1024, 1024), (200, 4096, 720)]:
        cfg, bm, bn, splits = plan(M, N, K)
        assert (bm, bn, splits) == (64, 64, 1), (M, N, K, cfg, bm, bn, splits)
    assert plan(256, 768, 3072, 4)[1:] == (64, 64, 4)
    for M, N, K in [(8192, 2304, 768), (8192, 768, 768), (8192, 768, 3072)]:
        assert plan(M, N, K)[1:] == (128, 192, 1), (M, N, K)
    assert plan(8192, 3072, 768)[3] == 1
    out = (C.c_uint32 * 4)()
    assert lib.sh_gemm_plan(0, 8, 8, 0, out) == -1


def test_gemm_tile_table_families(lib):
    """The tile-table index sets the GPU tests name (tests/conftest.py) are the library's families: register-staged
    (1), direct-to-LDS with the partial-slice variant (2), register epilogue (5), W^T operand (6), and the tiles with
    the in-workgroup split of two K ranges; out of range is -1."""
    from conftest import K2_CFGS, K5_CFGS, KG2_CFGS, REGSTAGED_CFGS, TILE_CFGS, WT_CFGS
    t = shops.tile_table()
    assert len(t) == TILE_CFGS == lib.sh_gemm_tile_count()
    fam = lambda f: tuple(i for i, r in enumerate(t) if r["family"] == f)   # noqa: E731
    assert (fam(1), fam(2), fam(5), fam(6)) == (REGSTAGED_CFGS, K2_CFGS, K5_CFGS, WT_CFGS)
    assert tuple(i for i, r in enumerate(t) if r["kg2"]) == KG2_CFGS
    assert all(t[i]["reg"] for i in K5_CFGS) and all(t[i]["ktail"] for i in K2_CFGS)
    assert all(r["wt"] == (i in WT_CFGS) for i, r in enumerate(t))
    assert all(r["bm"] % 64 == 0 and r["bn"] % 64 == 0 and r["threads"] in (256, 512, 768) for r in t)
    out = (C.c_uint32 * 8)()
    assert lib.sh_gemm_tile_info(TILE_CFGS, out) == -1
    assert lib.sh_gemm_tile_info(0, None) == -1


def test_gemm_plan_reports_the_launched_split_count(lib):
    """sh_gemm_plan reports the split count the launch runs: each K range is a whole number of 64-k slices
    (kps = 64 ceil(ceil(K / s) / 64)) and no trailing range is empty, so a request for more splits than K has
    64-k slices, or one that would leave an empty range, reports cdiv(K, kps)."""
    import ctypes as C

    def plan(M, N, K, splits):
        out = (C.c_uint32 * 4)()
        assert lib.sh_gemm_plan(M, N, K, splits, out) == 0
        return out[3]

    def launched(K, s):
        slices = -(-K // 64)
        s = max(1, min(s, slices))
        kps = 64 * -(-(-(-K // s)) // 64)
        return -(-K // kps)
    assert plan(256, 256, 256, 16) == 4            # 4 slices of 64: at most 4 ranges
    assert plan(256, 768, 768, 5) == 4             # kps = 192: ranges of 192, 192, 192, 192
    assert plan(256, 768, 768, 7) == 6             # kps = 128
    for K in (64, 192, 256, 720, 768, 3072):
        for s in range(1, 20):
            assert plan(256, 768, K, s) == launched(K, s), (K, s)


def test_prefetch_argument_errors_without_gpu(lib):
    assert lib.sh_prefetch(0, 64) == -1
    assert shops.last_error()[0] == -1
    assert lib.sh_prefetch(0, 0) == 0                    # an empty range is nothing to do, whatever its address


def test_dma_copy_argument_errors_without_gpu(lib):
    lib.sh_last_error()
    lib.sh_dma_copy(0, 1 << 20, 64)                    # NULL destination: refused before any HIP call
    assert lib.sh_last_error() == -1
    lib.sh_dma_copy(0, 0, 0)                           # nothing to copy: no error
    assert lib.sh_last_error() == 0
