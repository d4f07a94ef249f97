"""sh_gemm_splitk_noalloc (the entry point that allocates nothing) against sh_gemm_splitk through the C ABI: the
same kernels and summation order, so the same bits, on two calls in a row (the second smaller, so the shared
scratch array holds the first call's partials when it starts), both within tolerance of the oracle, and the
size limit refused before any GPU work."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import codes, to_dev, to_np
from oracle import refs
from softhier_mlir_amd import data, shops

pytestmark = pytest.mark.gpu
A = shops.addr


def _pair(lib, M, N, K, splits, seed):
    import torch
    x = data.uniform(M, K, seed)
    w = (data.uniform(K, N, seed + 1).astype(np.float32) / np.sqrt(K)).astype(np.float16)
    X, W = to_dev(x), to_dev(w)
    Zr = torch.empty((M, N), dtype=torch.float16, device="cuda")
    Zn = torch.full((M, N), 5.0, dtype=torch.float16, device="cuda")
    assert lib.sh_gemm_splitk(A(X), A(W), A(Zr), M, N, K, K, N, N, None, splits, shops.SH_ALL) == 0, shops.last_error()
    assert lib.sh_gemm_splitk_noalloc(A(X), A(W), A(Zn), M, N, K, K, N, N, None, splits, shops.SH_ALL) == 0, shops.last_error()
    return x, w, Zr, Zn


def test_noalloc_splitk_matches_splitk_on_two_calls(lib, gpu):
    import torch
    first = _pair(lib, 512, 1536, 3072, 4, 301)              # 4 x 512 x 1536 x 4 B = 12 MiB of partials
    torch.cuda.synchronize()
    second = _pair(lib, 256, 768, 3072, 4, 303)              # 3 MiB: the scratch still holds the first call's partials
    for x, w, Zr, Zn in (first, second):
        assert np.array_equal(codes(Zn), codes(Zr))
        bad, err, _ = refs.close(to_np(Zn), refs.gemm(x, w))
        assert bad == 0, err


def test_noalloc_splitk_scratch_boundary(lib, gpu):
    """The 16 MiB limit applies to launches that write fp32 partials: 4 K ranges of a 1024 x 1024 output need exactly
    16 MiB and run (the bits of sh_gemm_splitk); 8 ranges need 32 MiB and are refused before any GPU work; two equal
    K ranges run in one workgroup and write no partials, so a 1024 x 4096 output (32 MiB as partials) runs too."""
    import torch
    x, w, Zr, Zn = _pair(lib, 1024, 1024, 1024, 4, 311)
    assert np.array_equal(codes(Zn), codes(Zr))
    assert refs.close(to_np(Zn), refs.gemm(x, w))[0] == 0
    X, W = to_dev(x), to_dev(w)
    Z = torch.full((1024, 1024), 3.0, dtype=torch.float16, device="cuda")
    assert lib.sh_gemm_splitk_noalloc(A(X), A(W), A(Z), 1024, 1024, 1024, 1024, 1024, 1024, None, 8, shops.SH_ALL) == -1
    assert shops.last_error()[0] == -1
    torch.cuda.synchronize()
    assert (to_np(Z) == 3.0).all()                           # nothing ran
    x, w, Zr, Zn = _pair(lib, 1024, 4096, 1024, 2, 313)
    assert np.array_equal(codes(Zn), codes(Zr))
    assert refs.close(to_np(Zn), refs.gemm(x, w))[0] == 0
