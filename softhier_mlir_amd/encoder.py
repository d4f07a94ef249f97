"""SigLIP-B/ViT pre-LN encoder layer as a sequence of softhier-ops calls (the caller side of the boundary).

The op sequence is the reference's (softhier_mlir/frontend/siglip.py:133-168; the same calls a generated
main.c makes, tests/gvsoc/siglip_layer/main.c:64-127), on B sequences stacked as [B*S, D] rows:

    LN1 -> Q/K/V GEMM + bias -> 12-head attention -> out-proj GEMM + bias -> residual add -> LN2
        -> FFN-up GEMM + bias -> GELU -> FFN-down GEMM + bias -> residual add

`sequence="reference"` issues exactly those library calls (sh_layernorm, sh_gemm, sh_add_bias, sh_attention per
sequence, sh_add, sh_gelu). `sequence="fused"` computes the same layer with the additive entry points:
one QKV GEMM against the concatenated [D, 3D] weight with the bias in its epilogue, one batched attention
over q/k/v views of the QKV buffer (ld = 3D), and GEMM epilogues that add the bias, apply GELU or add the
residual, which removes five row-op round trips through HBM. Each LayerNorm is folded into the GEMM that reads
it: the GEMM multiplies the raw rows by W' = r16(gamma W) and its epilogue forms r (x W') - r mu c + d with
c = 1^T W', d = beta^T W + b (sh_ln_fold, once per weight), which is LN(x) W + b. The row statistics (mu, r) come
from the GEMM that stored the rows: out-proj and FFN-down write (sum, M2) pairs of every 32 columns of each output
row from their registers (sh_gemm_epi.stats_out), and the next QKV / FFN-up GEMM combines them. So a layer of
the stack is five launches (QKV, attention, out-proj, FFN-up, FFN-down); a layer whose input has no such
partials (the first) starts with sh_row_stats. Both sequences match the numpy oracle within the fp16 tolerance
(the fused epilogues round once where the reference rounds twice, and the fold rounds gamma W where the reference
rounds LN(x)).

Buffers are torch tensors (allocation only); every computation is a libshops.so call.
"""
from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass

import torch

from softhier_mlir_amd import shops

PARAM_NAMES = ("wq", "wk", "wv", "wo", "w1", "w2", "bq", "bk", "bv", "bo", "b1", "b2", "g1", "be1", "g2", "be2")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        code, msg = shops.last_error()
        raise RuntimeError(f"{what} failed with {rc}: {msg}")


@dataclass
class LayerParams:
    """fp16 device tensors of one layer; `wqkv` / `bqkv` are the concatenated Q|K|V weight and bias."""
    t: dict

    @classmethod
    def from_host(cls, p: dict, device: str = "cuda") -> "LayerParams":
        t = {nm: torch.as_tensor(p[nm]).to(device=device, dtype=torch.float16).contiguous() for nm in PARAM_NAMES}
        t["wqkv"] = torch.cat([t["wq"], t["wk"], t["wv"]], dim=1).contiguous()
        t["bqkv"] = torch.cat([t["bq"], t["bk"], t["bv"]], dim=1).contiguous()
        return cls(t)

    def __getitem__(self, k):
        return self.t[k]

    def fold(self, lib) -> None:
        """The weight side of both LayerNorm folds (sh_ln_fold, enqueued on the library stream), once: `wqkv_ln`,
        `cqkv`, `dqkv` for LN1 -> QKV and `w1_ln`, `c1`, `d1` for LN2 -> FFN-up (fp16 W', fp32 c and d). The weights
        the fused layer reads after its attention (`wo`, `w1_ln`, `w2`) then sit back to back in one allocation,
        `tail`, which the stack reads into the caches during attention as one range."""
        if "w1_ln" in self.t:
            return
        A = shops.addr
        wo, w1, w2 = self.t["wo"], self.t["w1"], self.t["w2"]
        tail = torch.empty(wo.numel() + w1.numel() + w2.numel(), dtype=torch.float16, device=wo.device)
        n0, n1 = wo.numel(), wo.numel() + w1.numel()
        self.t["wo"] = tail[:n0].view(wo.shape)
        self.t["wo"].copy_(wo)
        self.t["w2"] = tail[n1:].view(w2.shape)
        self.t["w2"].copy_(w2)
        self.t["tail"] = tail
        for w, g, be, b, tag in (("wqkv", "g1", "be1", "bqkv", "qkv"), ("w1", "g2", "be2", "b1", "1")):
            W = self.t[w]
            K, N = W.shape
            wp = tail[n0:n1].view(W.shape) if tag == "1" else torch.empty_like(W)
            c = torch.empty(N, dtype=torch.float32, device=W.device)
            d = torch.empty(N, dtype=torch.float32, device=W.device)
            lib.sh_last_error()                  # reads and clears: the check below sees this call's status only
            lib.sh_ln_fold(A(wp), A(c), A(d), A(W), A(self.t[g]), A(self.t[be]), A(self.t[b]), K, N, N, N)
            _check(lib.sh_last_error(), "sh_ln_fold " + w)
            self.t[w + "_ln"], self.t["c" + tag], self.t["d" + tag] = wp, c, d


class Encoder:
    """Runs layers on a [B*S, D] fp16 activation buffer; scratch buffers are allocated once per (B, S)."""

    def __init__(self, D: int = 768, F: int = 3072, H: int = 12, eps: float = 1e-6, device: str = "cuda"):
        self.D, self.F, self.H, self.eps, self.device = D, F, H, eps, device
        self.lib = shops.load()
        self.lib.sh_init()
        self._bufs: dict = {}
        self._pingpong: torch.Tensor | None = None   # the stack's second activation buffer (outside _bufs)
        self._plans: dict = {}               # fused-layer call lists by argument set (a stack has one per layer)
        self.gemm_cfg = shops.cfg()          # tile hints 256^3 (library default), as the reference's default policy
        self.row_partials = True             # False: sh_row_stats before each folded GEMM (seven launches a layer)
        self.tap = None                      # optional tap(name) -> context manager around each op (timing)
        self.prefetch = True                 # stacks: a layer's later weights read into the caches by its attention

    def _op(self, name: str):
        return self.tap(name) if self.tap is not None else contextlib.nullcontext()

    def buffers(self, rows: int) -> dict:
        if self._bufs.get("rows") != rows:
            z = lambda c: torch.empty((rows, c), dtype=torch.float16, device=self.device)  # noqa: E731
            D, F = self.D, self.F
            self._plans = {}
            self._bufs = {"rows": rows, "ln1": z(D), "qkv": z(3 * D), "q": z(D), "k": z(D), "v": z(D), "o": z(D),
                          "ao": z(D), "h": z(D), "ln2": z(D), "f1": z(F), "g": z(F), "f2": z(D),
                          "st1": torch.empty((rows, 2), dtype=torch.float32, device=self.device),
                          "st2": torch.empty((rows, 2), dtype=torch.float32, device=self.device),
                          "pst_x": torch.empty((rows, D // 32, 2), dtype=torch.float32, device=self.device),
                          "pst_h": torch.empty((rows, D // 32, 2), dtype=torch.float32, device=self.device)}
        return self._bufs

    # -- the reference's call sequence (siglip.py:133-168) ------------------------------------------------
    def layer_reference(self, x: torch.Tensor, out: torch.Tensor, p: LayerParams, B: int, S: int) -> torch.Tensor:
        L, A = self.lib, shops.addr
        D, F, H, rows = self.D, self.F, self.H, B * S
        b = self.buffers(rows)
        ALL = shops.SH_ALL
        cfg = self.gemm_cfg
        L.sh_layernorm(A(b["ln1"]), A(x), A(p["g1"]), A(p["be1"]), rows, D, D, self.eps, ALL)
        for dst, w, bias in (("q", "wq", "bq"), ("k", "wk", "bk"), ("v", "wv", "bv")):
            _check(L.sh_gemm(A(b["ln1"]), A(p[w]), A(b[dst]), rows, D, D, D, D, D, cfg, ALL), "sh_gemm " + dst)
            L.sh_add_bias(A(b[dst]), A(b[dst]), A(p[bias]), rows, D, D, ALL)
        scale = 1.0 / math.sqrt(D // H)
        for s in range(B):                   # the reference has no batch: one sh_attention call per sequence
            off = s * S * D
            _check(L.sh_attention(A(b["q"], off), A(b["k"], off), A(b["v"], off), A(b["o"], off), S, D, H, D, D, D, D, scale, ALL),
                   "sh_attention")
        _check(L.sh_gemm(A(b["o"]), A(p["wo"]), A(b["ao"]), rows, D, D, D, D, D, cfg, ALL), "sh_gemm wo")
        L.sh_add_bias(A(b["ao"]), A(b["ao"]), A(p["bo"]), rows, D, D, ALL)
        L.sh_add(A(b["h"]), A(x), A(b["ao"]), rows, D, D, ALL)
        L.sh_layernorm(A(b["ln2"]), A(b["h"]), A(p["g2"]), A(p["be2"]), rows, D, D, self.eps, ALL)
        _check(L.sh_gemm(A(b["ln2"]), A(p["w1"]), A(b["f1"]), rows, F, D, D, F, F, cfg, ALL), "sh_gemm w1")
        L.sh_add_bias(A(b["f1"]), A(b["f1"]), A(p["b1"]), rows, F, F, ALL)
        L.sh_gelu(A(b["g"]), A(b["f1"]), rows, F, F, ALL)
        _check(L.sh_gemm(A(b["g"]), A(p["w2"]), A(b["f2"]), rows, D, F, F, D, D, cfg, ALL), "sh_gemm w2")
        L.sh_add_bias(A(b["f2"]), A(b["f2"]), A(p["b2"]), rows, D, D, ALL)
        L.sh_add(A(out), A(b["h"]), A(b["f2"]), rows, D, D, ALL)
        return out

    # -- fused sequence (additive entry points) ------------------------------------------------------------
    def _fused_plan(self, x: torch.Tensor, out: torch.Tensor, p: LayerParams, B: int, S: int, x_parts: bool,
                    pf: tuple | None = None) -> list:
        """The layer's library calls with every argument converted once: (op name, function, args, what).
        x_parts: the row partials of x are in the `pst_x` buffer (written by the GEMM that stored x).
        pf: two (address, bytes) ranges the attention call reads into the caches (sh_attention_batched_prefetch)."""
        p.fold(self.lib)
        x_parts = x_parts and self.row_partials
        key = ((x.data_ptr(), out.data_ptr(), B, S, x_parts, self.row_partials, pf)
               + tuple(t.data_ptr() for t in p.t.values()))
        hit = self._plans.get(key)
        if hit is not None:
            return hit
        L, A = self.lib, shops.addr
        D, F, H, rows = self.D, self.F, self.H, B * S
        b = self.buffers(rows)
        cfg = self.gemm_cfg
        D3 = 3 * D
        qkv = b["qkv"]
        F32 = shops.SH_BIAS_FP32
        parts = D // 32
        sp = (lambda t: A(t)) if self.row_partials else (lambda t: 0)  # noqa: E731  (row partials written or not)
        calls = []
        if x_parts:
            ln1 = dict(ln_stats=A(b["pst_x"]), ln_parts=parts, ln_eps=self.eps)
        else:
            calls.append(("ln1", L.sh_row_stats, (A(b["st1"]), A(x), rows, D, D, self.eps), None))
            ln1 = dict(ln_stats=A(b["st1"]))
        calls += [
            ("qkv", L.sh_gemm_ex, (A(x), A(p["wqkv_ln"]), A(qkv), rows, D3, D, D, D3, D3, cfg,
                                   shops.epi(bias=A(p["dqkv"]), bias_fmt=F32, ln_c=A(p["cqkv"]), **ln1)),
             "sh_gemm_ex qkv"),
            ("attention", L.sh_attention_batched_prefetch if pf else L.sh_attention_batched,
             (A(qkv), A(qkv, D), A(qkv, 2 * D), A(b["o"]), B, S, D, H, D3, D3, D3, D, S * D3, S * D3, S * D3, S * D,
              1.0 / math.sqrt(D // H), 0) + ((pf[0][0], pf[0][1], pf[1][0], pf[1][1]) if pf else ()), "sh_attention_batched"),
            ("out_proj", L.sh_gemm_ex, (A(b["o"]), A(p["wo"]), A(b["h"]), rows, D, D, D, D, D, cfg,
                                        shops.epi(bias=A(p["bo"]), residual=A(x), ldr=D, stats_out=sp(b["pst_h"]))),
             "sh_gemm_ex wo"),
        ]
        if self.row_partials:
            ln2 = dict(ln_stats=A(b["pst_h"]), ln_parts=parts, ln_eps=self.eps)
        else:
            calls.append(("ln2", L.sh_row_stats, (A(b["st2"]), A(b["h"]), rows, D, D, self.eps), None))
            ln2 = dict(ln_stats=A(b["st2"]))
        calls += [
            ("ffn_up", L.sh_gemm_ex, (A(b["h"]), A(p["w1_ln"]), A(b["g"]), rows, F, D, D, F, F, cfg,
                                      shops.epi(bias=A(p["d1"]), bias_fmt=F32, act=shops.SH_ACT_GELU, ln_c=A(p["c1"]), **ln2)),
             "sh_gemm_ex w1"),
            ("ffn_down", L.sh_gemm_ex, (A(b["g"]), A(p["w2"]), A(out), rows, D, F, F, D, D, cfg,
                                        shops.epi(bias=A(p["b2"]), residual=A(b["h"]), ldr=D, stats_out=sp(b["pst_x"]))),
             "sh_gemm_ex w2"),
        ]
        if len(self._plans) >= 64:            # bounded: argument sets of retired buffers are dropped
            self._plans.clear()
        self._plans[key] = calls
        return calls

    def layer_fused(self, x: torch.Tensor, out: torch.Tensor, p: LayerParams, B: int, S: int,
                    x_parts: bool = False, prefetch: tuple | None = None) -> torch.Tensor:
        """One fused layer. x_parts=True: x was stored by the previous layer's FFN-down, whose row partials are in
        the encoder's `pst_x` buffer (the layer then skips sh_row_stats); the layer leaves out's in it.
        prefetch: two (address, bytes) ranges its attention reads into the caches (prefetch_ranges)."""
        for name, fn, args, what in self._fused_plan(x, out, p, B, S, x_parts, prefetch):
            with self._op(name):
                rc = fn(*args)
            if what is not None:
                _check(rc, what)
        return out

    def prefetch_ranges(self, p: LayerParams, nxt: "LayerParams | None") -> tuple:
        """The weights a fused layer reads after its attention (out-proj W, folded FFN-up W', FFN-down W: one
        allocation) and the next layer's folded QKV W', as two (address, bytes) ranges."""
        p.fold(self.lib)
        r0 = (shops.addr(p["tail"]), p["tail"].numel() * 2)
        if nxt is None:
            return r0, (0, 0)
        nxt.fold(self.lib)
        return r0, (shops.addr(nxt["wqkv_ln"]), nxt["wqkv_ln"].numel() * 2)

    def capture(self, x: torch.Tensor, out: torch.Tensor, p: LayerParams, B: int, S: int) -> "CapturedLayer":
        """Record one fused layer into a HIP graph (replay with `.replay()` on any stream). The layer runs once
        eagerly on the capture stream first, so buffers exist, every GEMM shape has its tile configuration settled
        and the stream's split-K workspace has its size; during capture the library enqueues on the capture
        stream, then returns to the stream it had. The returned object holds every buffer the graph addresses
        (the scratch set of this row count, x, out and the weights), so later calls with another row count,
        which replace the encoder's scratch set, cannot free memory the graph writes."""
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        prev = self.lib.sh_get_stream()
        try:
            with torch.cuda.stream(s):
                self.lib.sh_set_stream(s.cuda_stream)
                self.layer_fused(x, out, p, B, S)
                s.synchronize()
                with torch.cuda.graph(g, stream=s):
                    self.layer_fused(x, out, p, B, S)
        finally:
            self.lib.sh_set_stream(prev)
        torch.cuda.synchronize()
        return CapturedLayer(g, (dict(self.buffers(B * S)), x, out, p))

    @staticmethod
    def op_costs(B: int, S: int, D: int = 768, F: int = 3072, H: int = 12) -> dict:
        """Algorithmic FLOP and HBM bytes of each op of layer_fused (fp16 = 2 bytes; row statistics, row partials
        (8 bytes per 32 columns of a row) and the fold's c / d rows fp32; weights read once). "ln1" (sh_row_stats
        of the input) runs only in a layer whose input has no row partials (the first of a stack)."""
        M = B * S
        g = lambda m, n, k: 2 * m * n * k  # noqa: E731
        pb = 8 * M * (D // 32)              # row partials of one [M, D] activation
        return {
            "ln1": {"flop": 0, "bytes": 2 * M * D + 8 * M},
            "ln2": {"flop": 0, "bytes": 2 * M * D + 8 * M},   # (only with row_partials = False)
            "qkv": {"flop": g(M, 3 * D, D), "bytes": 2 * (M * D + D * 3 * D + M * 3 * D) + pb + 8 * 3 * D},
            "attention": {"flop": 4 * B * H * S * S * (D // H), "bytes": 2 * 4 * M * D},
            "out_proj": {"flop": g(M, D, D), "bytes": 2 * (M * D + D * D + D + 2 * M * D) + pb},
            "ffn_up": {"flop": g(M, F, D), "bytes": 2 * (M * D + D * F + M * F) + pb + 8 * F},
            "ffn_down": {"flop": g(M, D, F), "bytes": 2 * (M * F + F * D + D + 2 * M * D) + pb},
        }

    def forward(self, x: torch.Tensor, params: list[LayerParams], B: int, S: int, sequence: str = "fused",
                out: torch.Tensor | None = None) -> torch.Tensor:
        """len(params) layers; layer l reads layer l-1's output (siglip.py:168). Returns the last output."""
        step = self.layer_fused if sequence == "fused" else self.layer_reference
        n = len(params)
        out = out if out is not None else torch.empty_like(x)
        tmp = None
        if n > 1:                               # the ping-pong buffer persists, so the call plans stay valid
            tmp = self._pingpong
            if tmp is None or tmp.shape != x.shape or tmp.dtype != x.dtype or tmp.device != x.device:
                tmp = torch.empty_like(x)
                self._pingpong = tmp
        # a stack's weights do not all fit in the Infinity Cache next to its activations: each layer's attention reads
        # the layer's later weights and the next layer's QKV weight into the caches
        pre = sequence == "fused" and n > 1 and self.prefetch
        cur = x
        for i, p in enumerate(params):          # ping-pong so that the last layer writes `out`
            dst = out if (n - 1 - i) % 2 == 0 else tmp
            if sequence == "fused":
                rng = self.prefetch_ranges(p, params[i + 1] if i + 1 < n else None) if pre else None
                step(cur, dst, p, B, S, x_parts=i > 0, prefetch=rng)   # layer i > 0 reads the partials of layer i - 1
            else:
                step(cur, dst, p, B, S)
            cur = dst
        return out


class CapturedLayer:
    """A HIP graph of one fused layer and every buffer it addresses, kept alive together."""

    def __init__(self, graph: "torch.cuda.CUDAGraph", keep: tuple):
        self.graph = graph
        self._keep = keep

    def replay(self) -> None:
        self.graph.replay()


def flops_per_layer(B: int, S: int, D: int = 768, F: int = 3072) -> int:
    """2 B (4 S D^2 + 2 S D F + 2 S^2 D) (reference tests/gvsoc/run.py:315, counted as 2 FLOP per MAC)."""
    return 2 * B * (4 * S * D * D + 2 * S * D * F + 2 * S * S * D)
