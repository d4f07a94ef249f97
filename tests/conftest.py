"""Shared test setup: the `gpu` marker, device helpers and the library fixture.

`-m "not gpu"` tests run on any host (oracle pins, host logic, ABI exports, argument validation).
`-m gpu` tests call the HIP library through its C ABI on cuda:0 and compare with the oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


# Indices into the GEMM tile table (g_cfgs in sh_gemm.hip), by kernel family; tests/test_abi.py pins each set against
# sh_gemm_tile_info, so parametrised tests can name them at collection time without the library.
TILE_CFGS = 35
REGSTAGED_CFGS = tuple(range(0, 6))            # register-staged k_gemm (any alignment, any K; both W layouts)
K2_CFGS = tuple(range(6, 14))                  # direct-to-LDS k_gemm2 (also takes a partial last k-slice)
K5_CFGS = (14, 15, 16, 17, 32, 33, 34)         # direct-to-LDS k_gemm5, register epilogue (fold, row partials)
WT_CFGS = tuple(range(18, 32))                 # direct-to-LDS k_gemm6, W^T operand
KG2_CFGS = (16, 32)                            # k_gemm5 tiles with the in-workgroup split of two K ranges


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls libshops.so on cuda:0")


@pytest.fixture(scope="session")
def lib():
    """libshops.so bound through ctypes (imports torch first so both share one HIP runtime)."""
    import torch  # noqa: F401
    from softhier_mlir_amd import shops
    return shops.load()


@pytest.fixture(scope="session")
def gpu(lib):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    torch.cuda.init()
    lib.sh_init()
    return torch.device("cuda:0")


# Device tensors made by to_dev stay referenced until the test ends: library calls take raw addresses and run
# asynchronously, so a temporary (`A(to_dev(x))` as an argument) must not return its memory to torch's
# caching allocator before the kernels that read it have run.
_KEEP: list = []


@pytest.fixture(autouse=True)
def _keep_device_tensors_alive():
    from softhier_mlir_amd import shops
    if shops._lib is not None:          # sh_last_error reads and clears: no test sees an earlier test's error code
        shops._lib.sh_last_error()
    yield
    if _KEEP:
        import torch
        torch.cuda.synchronize()
        _KEEP.clear()


def to_dev(a: np.ndarray, dev="cuda:0"):
    """numpy fp16 (or uint16 codes) -> contiguous torch fp16 tensor on the GPU (kept alive for the test)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.float16)
    t = torch.from_numpy(a.astype(np.float16, copy=False)).to(dev)
    _KEEP.append(t)
    return t


def to_np(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def codes(t) -> np.ndarray:
    """fp16 tensor -> uint16 codes (bit-exact comparisons)."""
    return to_np(t).view(np.uint16)
