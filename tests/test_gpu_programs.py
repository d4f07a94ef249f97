"""Example softhier programs emitted with the HIP target (softhier_mlir_amd/programs/*.mlir, linked against
libshops.so by build()) run on the GPU as separate processes; their "<tag> r c hex" sample lines are checked
against the oracle on the same LCG inputs."""
from __future__ import annotations

import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import lcg, refs

pytestmark = pytest.mark.gpu
PROGS = Path(__file__).resolve().parents[1] / "softhier_mlir_amd" / "programs"


def run(name: str) -> tuple[str, dict]:
    exe = PROGS / f"{name}.exe"
    if not exe.exists():
        pytest.fail(f"{exe} is missing: build() emits and links the example programs")
    print(f"running {exe.name}", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    samples: dict = {}
    for m in re.finditer(r"^(\S+) (\d+) (\d+) ([0-9a-f]{4})$", r.stdout, re.M):
        samples.setdefault(m.group(1), []).append((int(m.group(2)), int(m.group(3)), int(m.group(4), 16)))
    assert "[Performance Counter]: Execution period is" in r.stdout
    return r.stdout, samples


def values(samples, tag, want: np.ndarray, nsamples: int, seed: int):
    got = samples[tag]
    assert [(i, j) for i, j, _ in got] == lcg.sample_positions(want.shape[0], want.shape[1], seed, nsamples)
    g = np.array([v for _, _, v in got], np.uint16).view(np.float16).astype(np.float32)
    w = np.array([want[i, j] for i, j, _ in got], np.float32)
    return g, w


def test_ops_check_program(gpu):
    _, smp = run("ops_check")
    x = lcg.fill_fp16(256, 768, 1, -16, 16, 0.125)
    g = lcg.fill_fp16(1, 768, 14, 2, 6, 0.25)
    be = lcg.fill_fp16(1, 768, 15, -4, 4, 0.125)
    qkv = lcg.fill_fp16(256, 2304, 21, -16, 16, 0.0625)
    y = refs.r16(refs.layernorm(x, g, be, 1e-6))
    kT = y.T.copy()
    s = refs.r16(refs.softmax(refs.r16(refs.gemm(y[:, 64:128], kT[64:128, :])), 0.125))
    ge = refs.r16(refs.gelu(y))
    ab = refs.r16(refs.add_bias(ge, be))
    ad = refs.r16(refs.add(x, ab))
    o = refs.attention(qkv[:, :768], qkv[:, 768:1536], qkv[:, 1536:], 12, 0.125)
    for tag, want, seed in (("Y", y, 31), ("S", s, 33), ("GE", ge, 34), ("AB", ab, 35), ("AD", ad, 36), ("O", o, 37)):
        got, w = values(smp, tag, want, 96, seed)
        bad, err, _ = refs.close(got, w)
        assert bad == 0, (tag, err)
    got, w = values(smp, "KT", kT, 96, 32)
    assert np.array_equal(got, w)                                      # transpose of the stored y: bit-exact


def test_siglip_layers_program(gpu):
    out, smp = run("siglip_layers")
    x = refs.siglip_input_lcg(256, 768)
    for L in range(2):
        x = refs.encoder_layer(x, refs.siglip_params_lcg(768, 3072, layer=L), 12)
        got, w = values(smp, f"OUT{L + 1}", x, 128, 205)
        bad, err, _ = refs.close(got, w)        # the north-star tolerance (tighter than run.py:963's 0.05 / 0.05)
        assert bad == 0, (L, err)
    assert re.search(r"^\[mark\] layer1 \d+$", out, re.M) and re.search(r"^\[mark\] layer2 \d+$", out, re.M)


def test_preload_gemm_program(gpu, tmp_path):
    """Operands arrive through a preload image (sh_preload_load: segments copied into the sh_hbm_addr arena)."""
    from softhier_mlir_amd import preload
    x = lcg.fill_fp16(256, 512, 51, -16, 16, 0.0625)
    w = lcg.fill_fp16(512, 384, 52, -16, 16, 0.03125)
    img = preload.write_image(tmp_path / "operands.elf", {4096: x, 266240: w, 856064: preload.sentinel()})
    exe = PROGS / "preload_gemm.exe"
    r = subprocess.run([str(exe), "--preload", str(img)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    smp = {}
    for m in re.finditer(r"^(\S+) (\d+) (\d+) ([0-9a-f]{4})$", r.stdout, re.M):
        smp.setdefault(m.group(1), []).append((int(m.group(2)), int(m.group(3)), int(m.group(4), 16)))
    got, want = values(smp, "Z", refs.gemm(x, w), 128, 41)
    bad, err, _ = refs.close(got, want)
    assert bad == 0, err


def test_preload_load_places_segments_bit_exact(lib, gpu, tmp_path):
    """sh_preload_load copies every segment to its arena offset; read back with the library's full dump."""
    from softhier_mlir_amd import preload, shops
    a = lcg.fill_fp16(33, 70, 61, -100, 100, 0.5)
    b = np.arange(1000, dtype=np.uint16).reshape(1, 1000)
    img = preload.write_image(tmp_path / "two.elf", {0x10000: a, 0x40000: b})
    assert lib.sh_preload_load(str(img).encode()) == 2
    for off, arr in ((0x10000, a.view(np.uint16)), (0x40000, b)):
        with shops.capture() as cap:
            lib.sh_test_dump_all(lib.sh_hbm_addr(off), arr.shape[0], arr.shape[1], arr.shape[1], b"P")
        got = np.zeros(arr.shape, np.uint16)
        for m in re.finditer(r"^P (\d+) (\d+) ([0-9a-f]{4})$", cap.text, re.M):
            got[int(m.group(1)), int(m.group(2))] = int(m.group(3), 16)
        assert np.array_equal(got, arr)
