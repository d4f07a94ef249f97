"""HIP target of the softhier emitter: a softhier-dialect program (MLIR text) -> a host C program that calls
libshops.so on one MI355X.

The reference lowers softhier-dialect modules to a `main.c` of softhier-ops calls for its RISC-V clusters
(softhier_mlir/backend/emit_c.py:327-430 op table, :567-570 phases, :672-703 program template), parsing the
module with xDSL. This target reads the same textual modules without xDSL (a line-oriented reader of the ops
the library implements) and emits the same calls, one per op, with the same argument derivation (operand
geometry from the memref types, views as address + element offset x 2, `cluster = -1` -> SH_ALL), so the
reference's translate tests (tests/filecheck/*_translate.mlir) check this output unchanged. The program is
a plain host `main()`: the library runs every call on the whole GPU, so there are no per-core stacks, and the
timed region is bracketed by `sh_barrier_global()` (stream drain) and the reference's timer line.

    python -m softhier_mlir_amd.emit_hip prog.mlir -o prog.c          # emit
    python -m softhier_mlir_amd.emit_hip prog.mlir --exe prog         # emit and link against libshops.so
    ./prog [--preload image.elf]                                      # run (image: softhier_mlir_amd/preload.py)

Ops outside the library (TCDM / RedMulE level, the expert and training families) make the reader raise.
"""
from __future__ import annotations

import argparse
import re
import shutil
import subprocess
import sys
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
INCLUDE = PKG.parent / "include"

_ELEM_BYTES = {"f16": 2, "bf16": 2, "f32": 4, "f64": 8, "i8": 1, "i16": 2, "i32": 4}
_FMT = {"fp16": "SH_FP16", "fp8": "SH_FP8", "int16": "SH_INT16", "int8": "SH_INT8"}
_XM_MODE = {"auto": "SH_XM_AUTO", "panel": "SH_XM_PANEL", "whole": "SH_XM_WHOLE"}


class EmitError(ValueError):
    pass


# ---- types and attributes -------------------------------------------------------------------------------
@dataclass
class MemRef:
    shape: tuple
    elem: str
    ld: int | None = None          # strides[0] of a strided layout
    eoff: int = 0                  # element offset of a strided layout

    @property
    def ebytes(self) -> int:
        return _ELEM_BYTES.get(self.elem, 2)

    @property
    def nbytes(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n * self.ebytes

    def geom(self) -> tuple[int, int, int, int]:
        """(rows, cols, ld, element offset); a 1-D memref is one row."""
        rows, cols = (1, self.shape[0]) if len(self.shape) == 1 else (self.shape[0], self.shape[1])
        ld = self.ld if (self.ld is not None and len(self.shape) > 1) else cols
        return rows, cols, ld, self.eoff


_MEMREF = re.compile(r"memref<([^,>]+?)x?(f16|bf16|f32|f64|i8|i16|i32)\s*(?:,\s*strided<\[([^\]]*)\](?:,\s*offset:\s*(\d+))?>)?\s*(?:,\s*\"[^\"]*\")?>")


def parse_memref(text: str) -> MemRef:
    m = _MEMREF.search(text)
    if not m:
        raise EmitError(f"not a memref type: {text!r}")
    dims = tuple(int(d) for d in m.group(1).rstrip("x").split("x") if d)
    ld = int(m.group(3).split(",")[0]) if m.group(3) else None
    return MemRef(dims, m.group(2), ld, int(m.group(4) or 0))


def _split_top(s: str, sep: str = ",") -> list[str]:
    """Split at `sep` outside <...>, [...], {...}, (...) and quotes."""
    out, depth, cur, quote = [], 0, [], False
    for ch in s:
        if ch == '"':
            quote = not quote
        elif not quote and ch in "<[{(":
            depth += 1
        elif not quote and ch in ">]})":
            depth -= 1
        if ch == sep and depth == 0 and not quote:
            out.append("".join(cur))
            cur = []
        else:
            cur.append(ch)
    if "".join(cur).strip():
        out.append("".join(cur))
    return [p.strip() for p in out]


def parse_attrs(text: str) -> dict:
    """`{k = v : type, unit_key, s = "str"}` -> {k: int | float | str | True}. f32 values are rounded to binary32."""
    body = text.strip()[1:-1].strip()
    out: dict = {}
    if not body:
        return out
    for item in _split_top(body):
        if "=" not in item:
            out[item.strip()] = True
            continue
        k, v = item.split("=", 1)
        k, v = k.strip(), v.strip()
        ty = None
        if not v.startswith('"') and " : " in v:
            v, ty = (p.strip() for p in v.rsplit(" : ", 1))
        if v.startswith('"'):
            out[k] = v[1:-1]
        elif v.startswith("["):
            out[k] = v                      # array attribute (kept as text; no op of this target reads one)
        elif ty in ("f32", "f16", "f64") or re.fullmatch(r"-?\d+\.\d*(e[-+]?\d+)?|-?\d+e[-+]?\d+", v):
            f = float(v)
            out[k] = float(np.float32(f)) if ty != "f64" else f
        else:
            out[k] = int(v)
    return out


def cfloat(v: float) -> str:
    """C float literal of an f32 attribute: the binary32 value printed as its shortest double repr, then 'f'."""
    return f"{float(np.float32(v))!r}f"


def cluster_arg(attrs: dict) -> str:
    c = attrs.get("cluster", 0)
    return "SH_SELF" if c == -2 else "SH_ALL" if c < 0 else str(c)


# ---- program structure ------------------------------------------------------------------------------------
@dataclass
class Op:
    name: str                       # e.g. "softhier.gemm", "scf.for", "arith.constant"
    result: str | None              # SSA name of the (single) result, or None
    operands: list                  # SSA names before '->' / 'into'
    outs: list                      # SSA names after '->' / 'into'
    attrs: dict
    types: str                      # trailing type signature text
    body: list = field(default_factory=list)      # nested ops (scf.for)
    extra: dict = field(default_factory=dict)


@dataclass
class Func:
    name: str
    attrs: dict
    ops: list


_STMT_START = re.compile(r"^(%[\w.$-]+(:\d+)?\s*=\s*)?([a-z_][\w]*\.[\w.]+|\})")   # "[%r =] dialect.op ..." or "}"


def _statements(lines: list[str]) -> list[str]:
    stmts: list[str] = []
    for ln in lines:
        s = ln.split("//", 1)[0].rstrip()
        if not s.strip():
            continue
        if _STMT_START.match(s.strip()) or not stmts:
            stmts.append(s.strip())
        else:
            stmts[-1] += " " + s.strip()
    return stmts


def _ssa_list(text: str) -> list[str]:
    return [t.strip() for t in text.split(",") if t.strip().startswith("%")]


def _parse_stmt(st: str) -> Op:
    result = None
    m = re.match(r"^(%[\w.$-]+)\s*=\s*(.*)$", st)
    if m:
        result, st = m.group(1), m.group(2)
    name = st.split(None, 1)[0]
    rest = st[len(name):].strip()
    if name == "arith.constant":
        v, ty = (p.strip() for p in rest.rsplit(":", 1))
        return Op(name, result, [], [], {"value": int(v)}, ty)
    if name in ("arith.addi", "arith.subi", "arith.muli", "arith.divui", "arith.remui"):
        lhs, rhs = (p.strip() for p in rest.rsplit(":", 1)[0].split(","))
        return Op(name, result, [lhs, rhs], [], {}, "index")
    if name == "scf.for":
        m = re.match(r"(%[\w.$-]+)\s*=\s*(%[\w.$-]+)\s+to\s+(%[\w.$-]+)\s+step\s+(%[\w.$-]+)\s*\{$", rest)
        if not m:
            raise EmitError(f"unsupported scf.for form: {st!r}")
        return Op(name, None, [m.group(2), m.group(3), m.group(4)], [], {}, "", extra={"iv": m.group(1)})
    if name in ("func.return", "scf.yield"):
        return Op(name, None, [], [], {}, "")
    if not name.startswith("softhier."):
        raise EmitError(f"unsupported op {name}")
    # softhier.<op> operands [-> outs | into %z] [{attrs}] [: types]
    attrs, types = {}, ""
    depth, colon = 0, -1
    for i, ch in enumerate(rest):            # the type signature starts at the first ':' outside {...}
        if ch == "{":
            depth += 1
        elif ch == "}":
            depth -= 1
        elif ch == ":" and depth == 0 and (i + 1 == len(rest) or rest[i + 1] == " "):
            colon = i
            break
    head, types = (rest[:colon], rest[colon + 1:].strip()) if colon >= 0 else (rest, "")
    a = head.find("{")
    if a >= 0:
        attrs = parse_attrs(head[a:head.rindex("}") + 1])
        head = head[:a]
    outs: list = []
    extra: dict = {}
    for kw in ("->", " into "):
        if kw in head:
            head, o = head.split(kw, 1)
            if " step " in o:                   # gemm ... into %z step %s: a per-step format table
                o, extra["step"] = o.split(" step ", 1)
            outs = _ssa_list(o)
            break
    return Op(name, result, _ssa_list(head), outs, attrs, types, extra=extra)


def parse(text: str) -> Func:
    """The first func.func of a module (softhier dialect, textual form)."""
    lines = text.splitlines()
    start = next((i for i, ln in enumerate(lines) if ln.strip().startswith("func.func")), None)
    if start is None:
        raise EmitError("no func.func in the module")
    hdr = lines[start].strip()
    m = re.match(r"func\.func\s+@([\w.$-]+)\s*\(\s*\)\s*(attributes\s*(\{.*\}))?\s*\{$", hdr)
    if not m:
        raise EmitError(f"unsupported func header: {hdr!r}")
    fattrs = parse_attrs(m.group(3)) if m.group(3) else {}
    stack: list[list] = [[]]
    for st in _statements(lines[start + 1:]):
        if st == "}":
            if len(stack) == 1:
                break                           # end of the function
            stack.pop()
            continue
        op = _parse_stmt(st)
        stack[-1].append(op)
        if op.name == "scf.for":
            stack.append(op.body)
    return Func(m.group(1), fattrs, stack[0])


# ---- emission -----------------------------------------------------------------------------------------------
class _Env:
    """SSA bindings: index expressions, buffers (space, C name / address expression, memref)."""

    def __init__(self) -> None:
        self.idx: dict = {}
        self.buf: dict = {}
        self.top_decls: list[str] = []
        self._nbuf = 0
        self._niv = 0

    def iexpr(self, v: str) -> str:
        if v not in self.idx:
            raise EmitError(f"{v} is not an index value")
        return self.idx[v]

    def new_buf(self) -> str:
        self._nbuf += 1
        return f"hb{self._nbuf}"

    def new_iv(self) -> str:
        self._niv += 1
        return f"i{self._niv}"

    def mt(self, v: str) -> MemRef:
        return self.buf[v][1]

    def name(self, v: str) -> str:
        return self.buf[v][0]

    def haddr(self, v: str) -> str:
        """HBM byte address of a (possibly viewed) buffer: base + element offset x element bytes."""
        mt = self.mt(v)
        return self.name(v) if mt.eoff == 0 else f"({self.name(v)} + {mt.eoff * mt.ebytes})"


def _declare_top(op: Op, env: _Env) -> None:
    mt = parse_memref(op.types)
    nm = env.new_buf()
    env.buf[op.result] = (nm, mt)
    shape = "x".join(str(d) for d in mt.shape)
    env.top_decls.append(f"    const uint64_t {nm} = sh_hbm_addr({op.attrs['offset']});  // {shape}x{mt.elem} HBM, {mt.nbytes} B")


def _gemm_cfg(op: Op) -> str:
    a = op.attrs
    return (f"{{ .tm = {a.get('tile_m', 0)}, .tn = {a.get('tile_n', 0)}, .tk = {a.get('tile_k', 0)}, "
            f".pipeline = {1 if 'pipeline' in a else 0}, .accumulate = {1 if 'accumulate' in a else 0}, "
            f".fmt = {_FMT.get(a.get('fmt', 'fp16'), 'SH_FP16')}, .l1_base = 0 }}")


_GUARD = "if (sh_cluster_id() == 0 && sh_is_first_core()) "


def _emit(ops: list, env: _Env, out: list, tag: str, ind: str) -> None:
    for op in ops:
        n, a = op.name, op.attrs
        if n == "arith.constant":
            env.idx[op.result] = str(a["value"])
        elif n in ("arith.addi", "arith.subi", "arith.muli", "arith.divui", "arith.remui"):
            sym = {"arith.addi": "+", "arith.subi": "-", "arith.muli": "*", "arith.divui": "/", "arith.remui": "%"}[n]
            env.idx[op.result] = f"({env.iexpr(op.operands[0])} {sym} {env.iexpr(op.operands[1])})"
        elif n in ("func.return", "scf.yield"):
            continue
        elif n == "scf.for":
            iv = env.new_iv()
            env.idx[op.extra["iv"]] = iv
            lb, ub, st = (env.iexpr(v) for v in op.operands)
            out.append(f"{ind}for (uint32_t {iv} = {lb}; {iv} < {ub}; {iv} += {st}) {{")
            _emit(op.body, env, out, tag, ind + "    ")
            out.append(f"{ind}}}")
        elif n == "softhier.hbm_buffer":
            if op.result in env.buf:
                continue                                   # top-level: declared with the function prologue
            mt = parse_memref(op.types)
            nm = env.new_buf()
            env.buf[op.result] = (nm, mt)
            shape = "x".join(str(d) for d in mt.shape)
            out.append(f"{ind}const uint64_t {nm} = sh_hbm_addr((uint64_t){a['offset']} + (uint64_t)({env.iexpr(op.operands[0])}) * "
                       f"{a.get('stride', 0)}u);  // {shape}x{mt.elem} HBM, {mt.nbytes} B, indexed")
        elif n == "softhier.view":
            mt = parse_memref(op.types.split("->", 1)[1])
            src = op.operands[0]
            nm = env.name(src)
            if len(op.operands) > 1:
                nm = f"({nm} + (uint64_t)({env.iexpr(op.operands[1])}) * {a.get('stride', 0) * mt.ebytes}u)"
            env.buf[op.result] = (nm, mt)
        elif n == "softhier.gemm":
            if "step" in op.extra or "fmt_steps" in a:       # a plain non-fp16 fmt is emitted; the library returns -1
                raise EmitError("softhier.gemm with a per-step format table belongs to the expert family (out of scope)")
            x, w = op.operands[0], op.operands[1]
            z = op.outs[0]
            m, k, ldx, _ = env.mt(x).geom()
            _, nn, ldw, _ = env.mt(w).geom()
            ldz = env.mt(z).geom()[2]
            args = f"{env.haddr(x)}, {env.haddr(w)}, {env.haddr(z)}, {m}, {nn}, {k}, {ldx}, {ldw}, {ldz}, &cfg"
            if "summa" in a:
                out.append(f"{ind}{{ sh_gemm_cfg cfg = {_gemm_cfg(op)};  // mesh-wide SUMMA")
                out.append(f"{ind}  sh_gemm_mesh({args}); }}")
            elif "xmcast" in a:
                mode = _XM_MODE[a["xmcast"] if isinstance(a["xmcast"], str) else "auto"]
                out.append(f"{ind}{{ sh_gemm_cfg cfg = {_gemm_cfg(op)};  // X-panel multicast, column slice per cluster")
                out.append(f"{ind}  sh_gemm_xmcast_ex({args}, {mode}); }}")
            else:
                out.append(f"{ind}{{ sh_gemm_cfg cfg = {_gemm_cfg(op)};")
                out.append(f"{ind}  sh_gemm({args}, {cluster_arg(a)}); }}")
        elif n == "softhier.hbm_fill":
            rows, cols = env.mt(op.operands[0]).shape
            out.append(f"{ind}sh_test_fill_const_fp16({env.name(op.operands[0])}, {rows}, {cols}, {cols}, {a['value_bits'] & 0xFFFF}u);")
        elif n == "softhier.hbm_fill_col_parity":
            rows, cols = env.mt(op.operands[0]).shape
            out.append(f"{ind}sh_test_fill_colparity_fp16({env.name(op.operands[0])}, {rows}, {cols}, {cols}, "
                       f"{a['even_bits'] & 0xFFFF}u, {a['odd_bits'] & 0xFFFF}u);")
        elif n == "softhier.hbm_check_const":
            rows, cols = env.mt(op.operands[0]).shape
            out.append(f"{ind}sh_test_check_const_fp16({env.name(op.operands[0])}, {rows}, {cols}, {cols}, "
                       f"{a['value_bits'] & 0xFFFF}u, {a['tol']}, \"{tag}\");")
        elif n == "softhier.hbm_fill_lcg":
            b = op.operands[0]
            rows, cols, ld, _ = env.mt(b).geom()
            out.append(f"{ind}{_GUARD}sh_test_fill_fp16({env.haddr(b)}, {rows}, {cols}, {ld}, {a['seed']}, {a['lo']}, {a['hi']}, "
                       f"{cfloat(a['scale'])});")
        elif n == "softhier.layernorm":
            x, g, be = op.operands[:3]
            y = op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            out.append(f"{ind}sh_layernorm({env.haddr(y)}, {env.haddr(x)}, {env.haddr(g)}, {env.haddr(be)}, {rows}, {cols}, {ld}, "
                       f"{cfloat(a['eps'])}, {cluster_arg(a)});")
        elif n == "softhier.rmsnorm":
            x, g = op.operands[:2]
            y = op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            out.append(f"{ind}sh_rmsnorm({env.haddr(y)}, {env.haddr(x)}, {env.haddr(g)}, {rows}, {cols}, {ld}, {cfloat(a['eps'])}, "
                       f"{cluster_arg(a)});")
        elif n == "softhier.softmax":
            x, y = op.operands[0], op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            if len(op.operands) > 1:
                mk = env.haddr(op.operands[1])
                out.append(f"{ind}sh_softmax_masked({env.haddr(y)}, {env.haddr(x)}, {rows}, {cols}, {ld}, {cfloat(a['scale'])}, {mk}, {mk}, "
                           f"{cluster_arg(a)});")
            else:
                out.append(f"{ind}sh_softmax_rows({env.haddr(y)}, {env.haddr(x)}, {rows}, {cols}, {ld}, {cfloat(a['scale'])}, {cluster_arg(a)});")
        elif n == "softhier.rope":
            x, tab = op.operands[:2]
            y = op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            ldt = env.mt(tab).geom()[2]
            out.append(f"{ind}sh_rope({env.haddr(y)}, {env.haddr(x)}, {env.haddr(tab)}, {rows}, {cols}, {ld}, {ldt}, {a['head_dim']}, "
                       f"{cluster_arg(a)});")
        elif n == "softhier.silu_mul":
            if len(op.operands) < 2:
                raise EmitError("softhier.silu_mul without a second operand is the expert family's kernel (out of scope)")
            xa, xb = op.operands[:2]
            y = op.outs[0]
            rows, cols, lda, _ = env.mt(xa).geom()
            if not (env.mt(y).geom()[2] == lda == env.mt(xb).geom()[2]):
                raise EmitError("softhier.silu_mul with distinct leading dimensions is the expert family's kernel (out of scope)")
            out.append(f"{ind}sh_silu_mul({env.haddr(y)}, {env.haddr(xa)}, {env.haddr(xb)}, {rows}, {cols}, {lda}, {cluster_arg(a)});")
        elif n == "softhier.scale":
            x, y = op.operands[0], op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            out.append(f"{ind}sh_scale({env.haddr(y)}, {env.haddr(x)}, {rows}, {cols}, {ld}, {cfloat(a['scale'])}, {cluster_arg(a)});")
        elif n == "softhier.pixel_shuffle":
            src, dst = op.operands[0], op.outs[0]
            rows, cols, _, _ = env.mt(src).geom()
            out.append(f"{ind}sh_pixel_shuffle({env.haddr(dst)}, {env.haddr(src)}, {int(round(rows ** 0.5))}, {cols}, {a['scale']}, "
                       f"{cluster_arg(a)});")
        elif n == "softhier.gelu":
            x, y = op.operands[0], op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            out.append(f"{ind}sh_gelu({env.haddr(y)}, {env.haddr(x)}, {rows}, {cols}, {ld}, {cluster_arg(a)});")
        elif n == "softhier.add":
            if "train" in a:
                raise EmitError("softhier.add {train} is the training family's kernel (out of scope)")
            xa, xb = op.operands[:2]
            y = op.outs[0]
            rows, cols, ld, _ = env.mt(xa).geom()
            out.append(f"{ind}sh_add({env.haddr(y)}, {env.haddr(xa)}, {env.haddr(xb)}, {rows}, {cols}, {ld}, {cluster_arg(a)});")
        elif n == "softhier.add_bias":
            x, bias = op.operands[:2]
            y = op.outs[0]
            rows, cols, ld, _ = env.mt(x).geom()
            out.append(f"{ind}sh_add_bias({env.haddr(y)}, {env.haddr(x)}, {env.haddr(bias)}, {rows}, {cols}, {ld}, {cluster_arg(a)});")
        elif n == "softhier.transpose":
            src, dst = op.operands[0], op.outs[0]
            rows, cols, lds, _ = env.mt(src).geom()
            ldd = env.mt(dst).geom()[2]
            out.append(f"{ind}sh_transpose({env.haddr(dst)}, {env.haddr(src)}, {rows}, {cols}, {lds}, {ldd}, {cluster_arg(a)});")
        elif n == "softhier.attention":
            q, k, v = op.operands[:3]
            o = op.outs[0]
            S, D, ldq, _ = env.mt(q).geom()
            ldk, ldv, ldo = env.mt(k).geom()[2], env.mt(v).geom()[2], env.mt(o).geom()[2]
            H = a["heads"]
            mask = op.operands[3] if len(op.operands) > 3 else None
            if mask is not None or "kv_heads" in a:
                hkv = a.get("kv_heads", H)
                mk = env.haddr(mask) if mask is not None else "0"
                out.append(f"{ind}sh_attention_gqa({env.haddr(q)}, {env.haddr(k)}, {env.haddr(v)}, {env.haddr(o)}, {S}, {D}, {H}, {hkv}, "
                           f"{ldq}, {ldk}, {ldv}, {ldo}, {cfloat(a['scale'])}, {mk}, {cluster_arg(a)});")
            else:
                qb = a.get("q_block", 0)
                out.append(f"{ind}sh_attention{'_q' if qb else ''}({env.haddr(q)}, {env.haddr(k)}, {env.haddr(v)}, {env.haddr(o)}, "
                           f"{S}, {D}, {H}, {ldq}, {ldk}, {ldv}, {ldo}, {cfloat(a['scale'])}, {cluster_arg(a)}{f', {qb}' if qb else ''});")
        elif n == "softhier.dump_samples":
            b = op.operands[0]
            rows, cols, ld, _ = env.mt(b).geom()
            if env.mt(b).elem == "f32":
                raise EmitError("f32 sample dumps belong to the training family (out of scope)")
            if len(op.operands) > 1:
                out.append(f"{ind}{_GUARD}sh_test_dump_samples_idx({env.haddr(b)}, {rows}, {cols}, {ld}, {a['seed']}, {a['n']}, "
                           f"\"{a['tag']}\", (uint32_t)({env.iexpr(op.operands[1])}));")
            else:
                out.append(f"{ind}{_GUARD}sh_test_dump_samples({env.haddr(b)}, {rows}, {cols}, {ld}, {a['seed']}, {a['n']}, \"{a['tag']}\");")
        elif n == "softhier.dump_all":
            b = op.operands[0]
            rows, cols, ld, _ = env.mt(b).geom()
            if len(op.operands) > 1:
                out.append(f"{ind}{_GUARD}sh_test_dump_all_idx({env.haddr(b)}, {rows}, {cols}, {ld}, \"{a['tag']}\", "
                           f"(uint32_t)({env.iexpr(op.operands[1])}));")
            else:
                out.append(f"{ind}{_GUARD}sh_test_dump_all({env.haddr(b)}, {rows}, {cols}, {ld}, \"{a['tag']}\");")
        elif n == "softhier.group_barrier":
            out.append(f"{ind}sh_barrier_global();")
        elif n == "softhier.preload_wait":
            out.append(f"{ind}sh_preload_wait({env.haddr(op.operands[0])});")
        elif n == "softhier.mark":
            if op.operands:
                out.append(f"{ind}{_GUARD}sh_printf(\"[mark] %s%u %u\\n\", \"{a['tag']}\", (uint32_t)({env.iexpr(op.operands[0])}), sh_cycles());")
            else:
                out.append(f"{ind}{_GUARD}sh_printf(\"[mark] %s %u\\n\", \"{a['tag']}\", sh_cycles());")
        else:
            raise EmitError(f"{n} has no softhier-ops call in this library")


_PROLOGUE = ("softhier.hbm_fill", "softhier.hbm_fill_col_parity", "softhier.hbm_fill_lcg", "softhier.preload_wait")
_STRUCTURAL = ("softhier.hbm_buffer", "softhier.view", "arith.constant", "arith.addi", "arith.subi", "arith.muli",
               "arith.divui", "arith.remui", "func.return")


def _base(v: str, defs: dict) -> str:
    while v in defs and defs[v].name == "softhier.view":
        v = defs[v].operands[0]
    return v


def _operands_deep(op: Op) -> list:
    out = list(op.operands) + list(op.outs)
    for inner in op.body:
        out.extend(_operands_deep(inner))
    return out


def _phase(op: Op, later: list, defs: dict) -> str:
    """Test inputs and the preload wait run before the timer; whole-buffer checks after it; a sample dump moves
    after the timer unless a later op touches its buffer (a reused residual stream is dumped in place)."""
    if op.name in _PROLOGUE:
        return "inputs"
    if op.name == "softhier.hbm_check_const":
        return "checks"
    if op.name == "softhier.dump_samples":
        base = _base(op.operands[0], defs)
        for lo in later:
            if lo.name in ("softhier.dump_samples", "softhier.hbm_check_const"):
                continue
            if any(_base(v, defs) == base for v in _operands_deep(lo)):
                return "kernel"
        return "checks"
    return "kernel"


def _defs(ops: list, out: dict | None = None) -> dict:
    out = {} if out is None else out
    for op in ops:
        if op.result:
            out[op.result] = op
        _defs(op.body, out)
    return out


def emit_phase(fn: Func, phase: str | None) -> str:
    try:
        return _emit_phase(fn, phase)
    except KeyError as e:
        raise EmitError(f"{e.args[0]} is not defined where it is used (or names an unsupported form)") from None


def _emit_phase(fn: Func, phase: str | None) -> str:
    env = _Env()
    for op in fn.ops:
        if op.name == "softhier.hbm_buffer" and not op.operands:
            _declare_top(op, env)
    defs = _defs(fn.ops)
    ops = [op for i, op in enumerate(fn.ops)
           if phase is None or op.name in _STRUCTURAL or _phase(op, fn.ops[i + 1:], defs) == phase]
    body: list[str] = []
    _emit(ops, env, body, fn.name.upper(), "    ")
    return "\n".join(env.top_decls + body)


_PROGRAM = '''\
// Generated by softhier_mlir_amd.emit_hip (softhier dialect -> softhier-ops calls on the HIP library). Do not edit.
// Usage: ./prog [--preload image.elf]   (an image in the reference's preload format, loaded into the HBM arena)
#include <string.h>
#include "sh_ops.h"

static void {name}_inputs(void) {{   // test inputs / preload wait (not timed)
{inputs}
}}

static void {name}(void) {{
{kernel}
}}

static void {name}_checks(void) {{   // test outputs (not timed)
{checks}
}}

int main(int argc, char **argv) {{
    sh_init();
    for (int i = 1; i + 1 < argc; ++i)
        if (strcmp(argv[i], "--preload") == 0 && sh_preload_load(argv[i + 1]) < 0) {{ sh_eoc(1); return 1; }}
    {name}_inputs();
    sh_barrier_global();
    sh_timer_start();
    {name}();
    sh_barrier_global();                 // the timed calls have run on the GPU
    sh_timer_end();
    {name}_checks();
    sh_barrier_global();
    const int rc = sh_last_error();
    sh_eoc(rc ? 1u : 0u);
    return rc ? 1 : 0;
}}
'''


def emit_hip(text: str) -> str:
    """The C program for the first func of a softhier-dialect module."""
    fn = parse(text)
    return _PROGRAM.format(name=fn.name, inputs=emit_phase(fn, "inputs"), kernel=emit_phase(fn, "kernel"),
                           checks=emit_phase(fn, "checks"))


def build_program(c_source: Path, exe: Path, lib_dir: Path = PKG) -> Path:
    """Compile an emitted program with the host C compiler and link it against libshops.so (rpath to `lib_dir`,
    relative to the executable when the library sits above it, so the pair can be moved together)."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no host C compiler found")
    lib = lib_dir / "libshops.so"
    if not lib.exists():
        raise RuntimeError(f"{lib} is missing: build the library first")
    try:
        rel = Path("$ORIGIN") / Path(*[".."] * (len(exe.resolve().parent.parts) - len(lib_dir.resolve().parts))) \
            if exe.resolve().parent.is_relative_to(lib_dir.resolve()) else lib_dir.resolve()
    except ValueError:
        rel = lib_dir.resolve()
    cmd = [cc, "-O2", "-std=c11", f"-I{INCLUDE}", str(c_source), f"-L{lib_dir}", "-lshops", f"-Wl,-rpath,{rel}",
           "-Wl,--allow-shlib-undefined", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("linking the emitted program failed:\n" + r.stdout + r.stderr)
    return exe


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("mlir")
    ap.add_argument("-o", "--output", help="C file to write (default: stdout)")
    ap.add_argument("--exe", help="also compile and link the program against libshops.so into this file")
    args = ap.parse_args(argv)
    src = emit_hip(Path(args.mlir).read_text())
    if args.output or args.exe:
        cpath = Path(args.output) if args.output else Path(args.exe).with_suffix(".c")
        cpath.write_text(src)
        if args.exe:
            build_program(cpath, Path(args.exe))
    else:
        sys.stdout.write(src)
    return 0


if __name__ == "__main__":
    sys.exit(main())
