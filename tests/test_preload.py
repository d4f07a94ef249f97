"""Preload images (the reference's HBM preload format, softhier_mlir/sim/preload.py:38-99) on the CPU: the image
layout, the writer's rules, and sh_preload_load's refusals (checked before any HIP call)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from softhier_mlir_amd import preload


def test_image_layout_and_round_trip(tmp_path):
    a = np.arange(300, dtype=np.float16).reshape(10, 30)
    b = np.arange(7, dtype=np.uint32)
    path = preload.write_image(tmp_path / "img.elf", {0x1000: a, 0x2000: b, 0x3000: preload.sentinel()})
    data = path.read_bytes()
    assert data[:4] == b"\x7fELF" and data[4] == 1 and data[5] == 1             # ELFCLASS32, little-endian
    e_type, e_machine = struct.unpack_from("<2H", data, 16)
    assert (e_type, e_machine) == (2, 243)                                      # EXEC, RISC-V (the GVSoC loader's)
    phoff, = struct.unpack_from("<I", data, 28)
    phentsize, phnum = struct.unpack_from("<2H", data, 42)
    assert (phoff, phentsize, phnum) == (52, 32, 3)
    segs = [struct.unpack_from("<8I", data, phoff + 32 * i) for i in range(phnum)]
    assert [s[3] for s in segs] == [preload.HBM_BASE + o for o in (0x1000, 0x2000, 0x3000)]   # paddr, offset order
    assert all(s[0] == 1 and s[1] % 64 == 0 for s in segs)                      # PT_LOAD, 64-byte aligned file offsets
    back = preload.read_image(path)
    assert back[0x1000] == a.tobytes() and back[0x2000] == b.tobytes()
    assert np.frombuffer(back[0x3000], np.uint32).tolist() == [0x5EEDC0DE] * 16


@pytest.mark.parametrize("arrays", [{0x800: np.zeros(4, np.float16)},                      # below 4 KiB
                                    {0x1010: np.zeros(4, np.float16)},                     # not 64-byte aligned
                                    {0x1000: np.zeros(64, np.float16), 0x1040: np.zeros(1, np.float16)}])  # overlap
def test_writer_rules(tmp_path, arrays):
    with pytest.raises(ValueError):
        preload.write_image(tmp_path / "bad.elf", arrays)


def test_loader_refuses_bad_images_before_touching_the_gpu(lib, tmp_path):
    assert lib.sh_preload_load(str(tmp_path / "missing.elf").encode()) == -1
    bad = tmp_path / "bad.elf"
    bad.write_bytes(b"not an elf image at all" * 4)
    assert lib.sh_preload_load(str(bad).encode()) == -1
    trunc = tmp_path / "trunc.elf"
    good = preload.write_image(tmp_path / "good.elf", {0x1000: np.zeros(64, np.float16)}).read_bytes()
    trunc.write_bytes(good[:60])                                                # program header cut off
    assert lib.sh_preload_load(str(trunc).encode()) == -1
    assert lib.sh_last_error() == -1
