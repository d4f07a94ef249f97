"""Build libshops.so (the softhier-ops C ABI, include/sh_ops.h) for gfx950 with hipcc, in-tree.

    python -m softhier_mlir_amd.build            # compile every csrc/*.hip, link softhier_mlir_amd/libshops.so

Each source is compiled to an object in parallel, then linked into one shared library. hipcc cross-compiles,
so this runs without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libshops.so"
OBJ = ROOT / "_build" / "obj"
ARCH = os.environ.get("SH_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU ops (the host pass warns that it does
# not know the feature; that is harmless).
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> tuple[Path, str]:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = [ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(noise))
    return obj, "\n".join(noise)


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libshops.so. Always rebuilds."""
    OBJ.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        results = list(ex.map(_compile, srcs))
    if verbose:
        for obj, log in results:
            if log.strip():
                print(f"[{obj.name}] {log}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


def build_programs() -> list[Path]:
    """Emit every example softhier program (programs/*.mlir) with the HIP target and link it against
    libshops.so: programs/<name>.gen.c and the executable programs/<name>.exe (host code only: gcc)."""
    from softhier_mlir_amd import emit_hip
    out = []
    for src in sorted((PKG / "programs").glob("*.mlir")):
        c = src.with_suffix(".gen.c")
        c.write_text(emit_hip.emit_hip(src.read_text()))
        out.append(emit_hip.build_program(c, src.with_suffix(".exe")))
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    for p in build_programs():
        print(p)
