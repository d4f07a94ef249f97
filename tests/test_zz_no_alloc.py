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


def test_noalloc_splitk_refuses_partials_beyond_its_scratch(lib, gpu):
    import torch
    M, N, K = 1024, 2048, 1024
    X = torch.zeros((M, K), dtype=torch.float16, device="cuda")
    W = torch.zeros((K, N), dtype=torch.float16, device="cuda")
    Z = torch.full((M, N), 3.0, dtype=torch.float16, device="cuda")
    # 4 x 1024 x 2048 x 4 B = 32 MiB of partials > 16 MiB
    assert lib.sh_gemm_splitk_noalloc(A(X), A(W), A(Z), M, N, K, K, N, N, None, 4, shops.SH_ALL) == -1
    assert shops.last_error()[0] == -1
    torch.cuda.synchronize()
    assert (to_np(Z) == 3.0).all()                           # nothing ran
    # 2 splits: 16 MiB exactly fits
    assert lib.sh_gemm_splitk_noalloc(A(X), A(W), A(Z), M, N, K, K, N, N, None, 2, shops.SH_ALL) == 0, shops.last_error()
    assert (to_np(Z) == 0.0).all()
