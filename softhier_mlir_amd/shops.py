"""ctypes binding of libshops.so: the softhier-ops C ABI declared in include/sh_ops.h.

Every function of the header is bound with its exact C signature, so Python calls read like the reference's C
drivers (tests/gvsoc/*/main.c) and the reference emitter's output: tensor arguments are 64-bit device byte
addresses (``addr(t)`` of a torch tensor, optionally offset by an element count for a strided view), leading
dimensions are element counts, and ``SH_ALL`` / ``cluster`` are accepted as in the reference.

The library must be built (``python -m softhier_mlir_amd.build``); loading fails loudly otherwise: there is no
fallback path.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libshops.so"
HEADER = PKG.parent / "include" / "sh_ops.h"

SH_ALL = 0xFFFFFFFF
SH_FP16, SH_FP8, SH_INT16, SH_INT8 = 0, 1, 2, 3
SH_EHIP = -3
SH_ACT_NONE, SH_ACT_GELU = 0, 1
SH_XM_AUTO, SH_XM_PANEL, SH_XM_WHOLE = 0, 1, 2
SH_LLM_PAD = 0xFFFF
SH_BIAS_FP16, SH_BIAS_FP32 = 0, 1
SH_MESH_P = 4


class sh_gemm_cfg(C.Structure):
    """runtime/sh_ops.h:54-60 of the reference: 7 x uint32, 0 = library default."""
    _fields_ = [("tm", C.c_uint32), ("tn", C.c_uint32), ("tk", C.c_uint32), ("pipeline", C.c_uint32),
                ("accumulate", C.c_uint32), ("fmt", C.c_uint32), ("l1_base", C.c_uint32)]


class sh_gemm_epi(C.Structure):
    """Fused GEMM epilogue of sh_gemm_ex (additive)."""
    _fields_ = [("bias", C.c_uint64), ("bias_fmt", C.c_uint32), ("act", C.c_uint32),
                ("residual", C.c_uint64), ("ldr", C.c_uint32), ("splits", C.c_uint32),
                ("ln_stats", C.c_uint64), ("ln_c", C.c_uint64), ("stats_out", C.c_uint64), ("ln_parts", C.c_uint32),
                ("ln_eps", C.c_float)]


u32, u64, i32, f32, i16 = C.c_uint32, C.c_uint64, C.c_int, C.c_float, C.c_uint16
_P = C.c_char_p
_SIGS: dict[str, tuple] = {
    # runtime wrappers
    "sh_init": (None, []), "sh_barrier_global": (None, []), "sh_barrier_cluster": (None, []),
    "sh_cluster_id": (u32, []), "sh_core_id": (u32, []), "sh_is_first_core": (i32, []), "sh_is_dm_core": (i32, []),
    "sh_num_clusters": (u32, []), "sh_timer_start": (None, []), "sh_timer_end": (None, []), "sh_eoc": (None, [u32]),
    "sh_cycles": (u32, []), "sh_hbm_addr": (u64, [u64]), "sh_hbm_malloc": (u64, [u32]), "sh_l1_size": (u32, []),
    "sh_preload_wait": (None, [u64]), "sh_preload_load": (i32, [_P]),
    # GEMM
    "sh_gemm": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg), u32]),
    "sh_gemm_mesh": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg)]),
    "sh_gemm_l1_bytes": (u32, [u32, u32, u32, C.POINTER(sh_gemm_cfg)]),
    "sh_gemm_xmcast": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg)]),
    "sh_gemm_xmcast_ex": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg), u32]),
    "sh_gemm_xmcast_l1_bytes": (u32, [u32, u32, u32, C.POINTER(sh_gemm_cfg), u32]),
    "sh_rmsnorm": (None, [u64, u64, u64, u32, u32, u32, f32, u32]),
    "sh_rope": (None, [u64, u64, u64, u32, u32, u32, u32, u32, u32]),
    "sh_silu_mul": (None, [u64, u64, u64, u32, u32, u32, u32]),
    "sh_softmax_masked": (None, [u64, u64, u32, u32, u32, f32, u64, u64, u32]),
    "sh_attention_head_masked": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, f32, u64, u32]),
    "sh_attention_gqa": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, u32, u32, f32, u64, u32]),
    "sh_pixel_shuffle": (None, [u64, u64, u32, u32, u32, u32]),
    "sh_dma_copy": (None, [u64, u64, u32]), "sh_prefetch": (i32, [u64, u64]),
    "sh_row_stats": (None, [u64, u64, u32, u32, u32, f32]),
    "sh_ln_fold": (None, [u64, u64, u64, u64, u64, u64, u64, u32, u32, u32, u32]),
    "sh_gemm_splitk": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg), u32, u32]),
    "sh_gemm_splitk_noalloc": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg), u32, u32]),
    "sh_gemm_ex": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg), C.POINTER(sh_gemm_epi)]),
    "sh_gemm_ex_wt": (i32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, C.POINTER(sh_gemm_cfg), C.POINTER(sh_gemm_epi)]),
    "sh_gemm_plan": (i32, [u32, u32, u32, u32, C.POINTER(C.c_uint32)]),
    "sh_gemm_tile_count": (i32, []), "sh_gemm_tile_info": (i32, [u32, C.POINTER(C.c_uint32)]),
    # row ops
    "sh_layernorm": (None, [u64, u64, u64, u64, u32, u32, u32, f32, u32]),
    "sh_layernorm_ld": (None, [u64, u64, u64, u64, u32, u32, u32, u32, f32]),
    "sh_softmax_rows": (None, [u64, u64, u32, u32, u32, f32, u32]),
    "sh_gelu": (None, [u64, u64, u32, u32, u32, u32]),
    "sh_add": (None, [u64, u64, u64, u32, u32, u32, u32]),
    "sh_add_bias": (None, [u64, u64, u64, u32, u32, u32, u32]),
    "sh_scale": (None, [u64, u64, u32, u32, u32, f32, u32]),
    "sh_transpose": (None, [u64, u64, u32, u32, u32, u32, u32]),
    # attention
    "sh_attention_head": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, f32, u32]),
    "sh_attention_q": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, u32, f32, u32, u32]),
    "sh_attention": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, u32, f32, u32]),
    "sh_attention_l1_bytes_q": (u32, [u32, u32, u32]), "sh_attention_l1_bytes": (u32, [u32, u32]),
    "sh_attention_q_block": (u32, [u32, u32, u32, u32]), "sh_attention_profile": (u32, [u32, u32, u32]),
    "sh_attention_batched": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, u32, u32, u64, u64, u64, u64, f32, u32]),
    "sh_attention_batched_prefetch": (i32, [u64, u64, u64, u64, u32, u32, u32, u32, u32, u32, u32, u32, u64, u64, u64, u64, f32,
                                            u32, u64, u64, u64, u64]),
    # test helpers
    "sh_test_fill_int_fp16": (None, [u64, u32, u32, u32, u32, i32, i32]),
    "sh_test_fill_fp16": (None, [u64, u32, u32, u32, u32, i32, i32, f32]),
    "sh_test_dump_samples": (None, [u64, u32, u32, u32, u32, u32, _P]),
    "sh_test_dump_samples_idx": (None, [u64, u32, u32, u32, u32, u32, _P, u32]),
    "sh_test_check_gemm": (u32, [u64, u64, u64, u32, u32, u32, u32, u32, u32, u32, f32, f32, _P]),
    "sh_test_fill_const_fp16": (None, [u64, u32, u32, u32, u32]),
    "sh_test_fill_colparity_fp16": (None, [u64, u32, u32, u32, u32, u32]),
    "sh_test_check_const_fp16": (u32, [u64, u32, u32, u32, u32, u32, _P]),
    "sh_test_dump_all": (None, [u64, u32, u32, u32, _P]),
    "sh_test_dump_all_idx": (None, [u64, u32, u32, u32, _P, u32]),
    "sh_fp16_to_f32": (f32, [i16]), "sh_f32_to_fp16": (i16, [f32]),
    # additive runtime
    "sh_last_error": (i32, []), "sh_last_error_str": (_P, []), "sh_set_stream": (None, [u64]), "sh_get_stream": (u64, []),
    "sh_stream_release": (i32, [u64]), "sh_stream_workspace_bytes": (u64, [u64]),
    "sh_timer_last_ns": (C.c_double, []), "sh_capture": (None, [i32]), "sh_captured": (u64, [C.c_void_p, u64]),
}
# variadic / function-pointer entry points: bound without a prototype
_UNTYPED = {"sh_printf", "sh_call_on_core_stack"}

_lib: C.CDLL | None = None


def load(path: str | Path | None = None) -> C.CDLL:
    """Load libshops.so once and bind every signature. Raises if the library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it with `python -m softhier_mlir_amd.build` (no fallback path exists)")
    lib = C.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def header_functions(header: Path = HEADER) -> list[str]:
    """Names of every function prototype declared in include/sh_ops.h (static inline helpers excluded)."""
    text = re.sub(r"/\*.*?\*/", " ", header.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    names = []
    for m in re.finditer(r"^\s*(?!static|typedef|#)[A-Za-z_][\w\s\*]*?\b(sh_\w+)\s*\(", text, flags=re.M):
        names.append(m.group(1))
    return sorted(set(names))


def cfg(tm: int = 0, tn: int = 0, tk: int = 0, pipeline: int = 1, accumulate: int = 0, fmt: int = SH_FP16,
        l1_base: int = 0) -> sh_gemm_cfg:
    return sh_gemm_cfg(tm, tn, tk, pipeline, accumulate, fmt, l1_base)


def epi(bias: int = 0, bias_fmt: int = SH_BIAS_FP16, act: int = SH_ACT_NONE, residual: int = 0, ldr: int = 0,
        splits: int = 1, ln_stats: int = 0, ln_c: int = 0, stats_out: int = 0, ln_parts: int = 0,
        ln_eps: float = 0.0) -> sh_gemm_epi:
    return sh_gemm_epi(bias, bias_fmt, act, residual, ldr, splits, ln_stats, ln_c, stats_out, ln_parts, ln_eps)


def addr(t, elem_offset: int = 0) -> int:
    """Device byte address of a torch tensor's storage start plus `elem_offset` elements (a strided view)."""
    return int(t.data_ptr()) + int(elem_offset) * t.element_size()


def tile_table() -> list[dict]:
    """The GEMM tile table (sh_gemm_tile_info of every entry, in index order)."""
    lib = load()
    keys = ("bm", "bn", "family", "threads", "wt", "reg", "kg2", "ktail")
    rows = []
    for i in range(lib.sh_gemm_tile_count()):
        out = (C.c_uint32 * 8)()
        if lib.sh_gemm_tile_info(i, out) != 0:
            raise RuntimeError(f"sh_gemm_tile_info({i}) failed")
        rows.append(dict(zip(keys, (int(v) for v in out))))
    return rows


def last_error() -> tuple[int, str]:
    lib = load()
    code = lib.sh_last_error()
    return code, (lib.sh_last_error_str() or b"").decode()


class capture:
    """Context manager: collect everything the library prints (sample dumps, timer lines) as a string."""

    def __enter__(self):
        load().sh_capture(1)
        self.text = ""
        return self

    def __exit__(self, *exc):
        lib = load()
        n = lib.sh_captured(None, 0)
        buf = C.create_string_buffer(int(n) + 1)
        lib.sh_captured(buf, n + 1)
        lib.sh_capture(0)
        self.text = buf.value.decode()
        return False
