"""Preload images: the reference's HBM preload format (softhier_mlir/sim/preload.py:38-99), written and read here
so that data prepared for the reference's `--preload` flow reaches the HIP library unchanged.

An image is a little-endian ELF32 whose PT_LOAD segments place raw array bytes at physical address
HBM_BASE + offset (offsets >= 4 KiB, 64-byte aligned, non-overlapping, written in offset order); the last
segment is a 64-byte sentinel of 16 x SENTINEL_MAGIC that `softhier.preload_wait` points at. On the GPU,
`sh_preload_load(path)` copies every segment into the `sh_hbm_addr` arena before the program runs, so the
sentinel wait reduces to a stream drain. Emitted programs take `--preload <image>`.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

HBM_BASE = 0xC0000000          # SH_PRELOAD_HBM_BASE in include/sh_ops.h
MIN_OFFSET = 0x1000
ALIGN = 64
SENTINEL_MAGIC = 0x5EEDC0DE
SENTINEL_WORDS = 16
_EM_RISCV, _PT_LOAD, _PF_RW = 243, 1, 6


def sentinel() -> np.ndarray:
    """The 64-byte end-of-preload marker as a [1, 32] fp16 array (raw bits: 16 x SENTINEL_MAGIC)."""
    return np.full(SENTINEL_WORDS, SENTINEL_MAGIC, np.uint32).view(np.float16).reshape(1, 2 * SENTINEL_WORDS)


def write_image(path: str | Path, arrays: dict[int, np.ndarray]) -> Path:
    """ELF32 image placing each array (raw little-endian bytes, row-major) at HBM_BASE + its byte offset."""
    items = sorted((int(o), np.ascontiguousarray(a)) for o, a in arrays.items())
    end = 0
    for off, a in items:
        if off < MIN_OFFSET or off % ALIGN or off < end:
            raise ValueError(f"segment at 0x{off:x}: offsets must be >= 0x{MIN_OFFSET:x}, {ALIGN}-byte aligned and not overlap")
        end = off + a.nbytes
    ehsize, phsize = 52, 32
    pos = -(-(ehsize + phsize * len(items)) // ALIGN) * ALIGN
    heads, body = [], []
    for off, a in items:
        heads.append(struct.pack("<8I", _PT_LOAD, pos, HBM_BASE + off, HBM_BASE + off, a.nbytes, a.nbytes, _PF_RW, ALIGN))
        pad = -a.nbytes % ALIGN
        body.append((pos, a.tobytes() + bytes(pad)))
        pos += a.nbytes + pad
    out = bytearray(pos)
    ident = b"\x7fELF" + bytes([1, 1, 1]) + bytes(9)
    out[0:ehsize] = ident + struct.pack("<2H5I6H", 2, _EM_RISCV, 1, HBM_BASE, ehsize, 0, 0, ehsize, phsize, len(items), 0, 0, 0)
    for i, h in enumerate(heads):
        out[ehsize + i * phsize:ehsize + (i + 1) * phsize] = h
    for p, b in body:
        out[p:p + len(b)] = b
    path = Path(path)
    path.write_bytes(bytes(out))
    return path


def read_image(path: str | Path) -> dict[int, bytes]:
    """{offset: raw bytes} of every PT_LOAD segment of an image."""
    data = Path(path).read_bytes()
    if data[:4] != b"\x7fELF" or data[4] != 1 or data[5] != 1:
        raise ValueError(f"{path} is not a little-endian ELF32 image")
    phoff, = struct.unpack_from("<I", data, 28)
    phentsize, phnum = struct.unpack_from("<2H", data, 42)
    out = {}
    for i in range(phnum):
        ptype, foff, _, paddr, size = struct.unpack_from("<5I", data, phoff + i * phentsize)
        if ptype == _PT_LOAD:
            out[paddr - HBM_BASE] = data[foff:foff + size]
    return out
