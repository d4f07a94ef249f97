"""Benchmark of the softhier-ops hot path on one MI355X: the SigLIP-B encoder layer (
B=32, S=256, D=768, 12 heads, FFN 3072, fp16, weights N(0, 0.02), biases zero, x ~ N(0, 1), seeded).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--sequence fused|reference] [--graph] [--no-cpu] [--no-rowops]

A step is one forward pass of one layer over the batch through libshops.so (inputs resident in HBM), its calls
launched one by one, as a layer runs inside the 12-layer stack: the fused layer (five launches) reads the rows
and the row partials the previous step stored (the first step computes the row statistics of the input itself);
`--row-stats` times the seven-launch variant with a row-statistics pass before each folded GEMM. `--graph`
records the fused layer (from the input's own statistics) once into a HIP graph and times replays of it instead.
Prints ONE JSON line with the whole-job TFLOP/s, the roofline of the dominant kernel (its call of the timed step
launched K times back to back between one HIP event pair on the library stream = the legacy null stream),
the per-op breakdown, the row-op HBM bandwidths at the batched shapes (cold: rotating buffer sets of >= 512 MiB;
each next to the library's streaming copy of the same bytes) and the numpy CPU baseline (the oracle's
restatement, timed on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "encoder-layer TFLOP/s fp16 (S=256,D=768,B=32); % MFMA peak; rowops HBM GB/s"
PEAK_TFLOPS = 2500.0        # MI355X dense fp16 MFMA
PEAK_GBS = 8000.0           # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sequence", default="fused", choices=["fused", "reference"])
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--seq", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true", help="skip the numpy CPU baseline")
    ap.add_argument("--no-rowops", action="store_true", help="skip the row-op bandwidth measurement")
    ap.add_argument("--graph", action="store_true",
                    help="replay a captured HIP graph of the layer instead of launching its kernels one by one")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the layer line: every BASELINE config on its own (time, parity, CPU oracle time), "
                         "one JSON line each")
    ap.add_argument("--row-stats", action="store_true",
                    help="fused layer with sh_row_stats before each folded GEMM (7 launches) instead of row partials")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the 12-layer stack and the S=1024 attention measurements")
    ap.add_argument("--library-gemm", action="store_true",
                    help="instead of the layer line: the four encoder GEMM shapes through sh_gemm_ex (plain and with the "
                         "layer's epilogue) next to torch.matmul (hipBLASLt), one JSON line")
    ap.add_argument("--torch-sdpa", action="store_true",
                    help="instead of the layer line: batched attention (B=32 S=256, B=8 S=1024, 12 heads of 64) through "
                         "sh_attention_batched next to torch's scaled_dot_product_attention (flash and memory-efficient "
                         "backends only), one JSON line")
    ap.add_argument("--torch-rowops", action="store_true",
                    help="instead of the layer line: the row ops at the batched shapes, cold, through the library next to "
                         "torch's own kernels for the same ops (layer_norm, softmax, tanh GELU, add, bias add, transpose "
                         "copy), one JSON line")
    ap.add_argument("--torch-layer", action="store_true",
                    help="instead of the layer line: the same encoder layer (weights, input, op order) as a torch eager "
                         "forward (layer_norm, linear = hipBLASLt, flash scaled_dot_product_attention, tanh GELU), timed as "
                         "the bench line times the library's, next to the library's fused layer, one JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 3 plain device copies of 512 MiB (a known-size kernel for scaling HBM counters)")
    ap.add_argument("--stack", action="store_true",
                    help="instead of the layer line: the 12-layer stack only (K forwards after W warm-up forwards), with "
                         "per-layer HIP-event times, one JSON line (for kernel traces of the stack)")
    ap.add_argument("--copy-curve", action="store_true",
                    help="instead of the layer line: device copy bandwidth from 1 MB to 1.6 GB, cold, for the library's "
                         "streaming copy and the HIP runtime's device-to-device copy, one JSON line")
    return ap.parse_args()


_WARM: dict = {}


def busy(torch, fn, seconds: float) -> None:
    """Untimed warm-up before a timed region: a large fp16 product (8192^3 through torch.matmul, ~1.5 ms a launch)
    back to back for `seconds` of wall time, then `fn` three times. On MI355X the same kernel runs up to ~20 %
    slower until the GPU has been busy for ~20 ms, and again after ~50 ms idle (the clocks follow sustained load):
    a few launches of a short kernel do not get there, and thousands of them would flood a kernel trace."""
    if "a" not in _WARM:
        g = torch.Generator(device="cuda").manual_seed(0)
        _WARM["a"] = torch.randn((8192, 8192), dtype=torch.float16, device="cuda", generator=g)
        _WARM["c"] = torch.empty_like(_WARM["a"])
    a, c = _WARM["a"], _WARM["c"]
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(4):
            torch.matmul(a, a, out=c)
        torch.cuda.synchronize()
    for _ in range(3):
        fn()
    torch.cuda.synchronize()


def traced_avg_us(op: str):
    """(kernel, average us per launch, {figure: us}) of `op` in the committed layer kernel trace
    (profiles/encoder_layer_b32_s256_kernel_trace.md, rocprofv3 --kernel-trace --stats): the `--stats` average over
    every launch of the kernel in the traced command (its `roofline_trace ... stats_avg_us` line), else the op's
    average in the timed layer steps; the trace's other figures for the op (in the timed steps, back to back) ride
    along. None without the file."""
    f = ROOT / "profiles" / "encoder_layer_b32_s256_kernel_trace.md"
    if not f.exists():
        return None
    kernel, avg, figs = None, None, {}
    for line in f.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == op and cells[3].isdigit():
            kernel, avg = cells[1].strip("`"), float(cells[4])
        if line.startswith(f"roofline_trace {op} "):
            name, val = line[len(f"roofline_trace {op} "):].split(":")
            figs[name.strip()] = float(val)
    if kernel is None:
        return None
    return kernel, figs.get("stats_avg_us", avg), figs


def counted_traffic(op: str):
    """HBM bytes per launch of `op` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by a
    known-size copy; profiles/*hbm_counters.md), or None when no summary covers the op."""
    for f in sorted((ROOT / "profiles").glob("*hbm_counters.md")):
        for line in f.read_text().splitlines():
            if line.startswith(f"traffic_bytes_per_launch {op}:"):
                return int(line.split(":")[1])
    return None


def rowops_bandwidth(lib, torch, B: int, S: int, D: int, F: int, H: int, reps: int = 3, scale: int = 1) -> dict:
    """Row ops at the batched shapes (scale = 1) or at `scale` times as many rows (the large-size table), cold:
    buffer sets rotated so that >= 512 MiB is touched between reuses (MI355X Infinity Cache = 256 MiB).
    Algorithmic bytes: each input read once, the output written once. The ceiling next to each op is the
    library's own streaming copy (sh_dma_copy) of the output's bytes."""
    from softhier_mlir_amd import shops
    A = shops.addr
    M = B * S * scale
    ops = {
        "layernorm": ((M, D), 2 * (2 * M * D + 2 * D)),
        "softmax": ((H * M, S), 2 * 2 * H * M * S),
        "gelu": ((M, F), 2 * 2 * M * F),
        "add": ((M, D), 2 * 3 * M * D),
        "add_bias": ((M, D), 2 * (2 * M * D + D)),
        "transpose": ((M, D), 2 * 2 * M * D),
    }
    out = {}
    g = torch.ones((1, max(D, F)), dtype=torch.float16, device="cuda")
    be = torch.zeros((1, max(D, F)), dtype=torch.float16, device="cuda")
    for name, ((r, c), nbytes) in ops.items():
        per_set = nbytes
        nsets = max(2, int((512 << 20) // per_set) + 1)
        sets = []
        for _ in range(nsets):
            x = torch.randn((r, c), dtype=torch.float16, device="cuda")
            y = torch.empty((c, r) if name == "transpose" else (r, c), dtype=torch.float16, device="cuda")
            b = torch.randn((r, c), dtype=torch.float16, device="cuda") if name == "add" else None
            sets.append((x, y, b))

        def run(x, y, b):
            if name == "layernorm":
                lib.sh_layernorm(A(y), A(x), A(g), A(be), r, c, c, 1e-6, shops.SH_ALL)
            elif name == "softmax":
                lib.sh_softmax_rows(A(y), A(x), r, c, c, 0.125, shops.SH_ALL)
            elif name == "gelu":
                lib.sh_gelu(A(y), A(x), r, c, c, shops.SH_ALL)
            elif name == "add":
                lib.sh_add(A(y), A(x), A(b), r, c, c, shops.SH_ALL)
            elif name == "add_bias":
                lib.sh_add_bias(A(y), A(x), A(g), r, c, c, shops.SH_ALL)
            else:
                lib.sh_transpose(A(y), A(x), r, c, c, r, shops.SH_ALL)

        def copy(x, y, b):
            lib.sh_dma_copy(A(y), A(x), 2 * r * c)

        def timed(fn):
            """(median us of single launches with events around each, us per launch of all sets back to back)"""
            busy(torch, lambda: [fn(*st) for st in sets], 0.15)
            times = []
            for _ in range(reps):
                for st in sets:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn(*st)
                    e1.record()
                    times.append((e0, e1))
            torch.cuda.synchronize()
            ms = sorted(a.elapsed_time(b) for a, b in times)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for st in sets:
                fn(*st)
            e1.record()
            torch.cuda.synchronize()
            return ms[len(ms) // 2] * 1e3, e0.elapsed_time(e1) * 1e3 / len(sets)

        us, us_b = timed(run)
        cus, cus_b = timed(copy)          # a device copy of the output's bytes: 2 x output bytes of traffic
        gbs = nbytes / (us * 1e-6) / 1e9
        cbytes = 2 * 2 * r * c
        out[name] = {"shape": [r, c], "bytes": nbytes, "us": round(us, 2), "GB/s": round(gbs, 1),
                     "frac": round(gbs / PEAK_GBS, 3), "us_batched": round(us_b, 2),
                     "GB/s_batched": round(nbytes / (us_b * 1e-6) / 1e9, 1),
                     "copy_GB/s": round(cbytes / (cus * 1e-6) / 1e9, 1),
                     "frac_of_copy": round(gbs / (cbytes / (cus * 1e-6) / 1e9), 3)}
        del sets
        torch.cuda.empty_cache()
    return out


def stack12(torch, enc, x, B: int, S: int, D: int, F: int, reps: int = 5, warmup: int = 1) -> dict:
    """The 12-layer stack (layer l reads layer l-1's output, weights of layer l seeded 100 + l),
    each layer's attention reading the layer's later weights and the next layer's QKV weight into the caches
    (sh_attention_batched_prefetch; `enc.prefetch = False`: not). `reps` 12-layer forwards and `reps` 1-layer
    forwards (layer 0 alone) are timed on the host clock between synchronisations, alternating; the steady per-layer
    time is their difference over 11 layers, which cancels the first layer's own costs (its input's row
    statistics, the launch latency after a synchronisation). Nothing is recorded between layers: an event on the
    library stream costs the next kernel a few microseconds."""
    from softhier_mlir_amd import data, encoder
    layers = [encoder.LayerParams.from_host(data.encoder_params(D, F, seed=100 + l)) for l in range(12)]
    y = torch.empty_like(x)
    for _ in range(max(1, warmup)):
        enc.forward(x, layers, B, S, out=y)             # warm-up (buffers, tile choices)
        enc.forward(x, layers[:1], B, S, out=y)
    busy(torch, lambda: enc.forward(x, layers, B, S, out=y), 0.25)

    def timed(ls):
        t0 = time.perf_counter()
        for _ in range(reps):
            enc.forward(x, ls, B, S, out=y)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / reps

    t12, t1 = [], []
    for _ in range(3):
        t12.append(timed(layers))
        t1.append(timed(layers[:1]))
    ms12, ms1 = min(t12), min(t1)
    flop = 12 * encoder.flops_per_layer(B, S, D, F)
    del layers, y
    return {"layers": 12, "ms_per_forward": round(ms12, 3), "TFLOP/s": round(flop / (ms12 * 1e-3) / 1e12, 1),
            "ms_one_layer_forward": round(ms1, 3), "us_per_layer_steady": round((ms12 - ms1) * 1e3 / 11, 1),
            "weight_prefetch": bool(enc.prefetch)}


def copy_curve(lib, torch) -> dict:
    """Device copy bandwidth against size, cold (buffer sets rotated over >= 512 MiB, twice the Infinity Cache):
    the library's streaming copy (sh_dma_copy) and the HIP runtime's device-to-device copy (torch copy_ =
    hipMemcpyAsync). Traffic = 2 x bytes (read + write); median of single launches with events around each."""
    from softhier_mlir_amd import shops
    A = shops.addr
    rows = []
    for mb in (1, 2, 4, 8, 16, 25, 32, 64, 100, 128, 256, 400, 512, 1024, 1600):
        n = mb << 20
        nsets = max(2, (512 << 20) // n + 1)
        sets = [(torch.empty(n // 2, dtype=torch.float16, device="cuda").fill_(1.0),
                 torch.empty(n // 2, dtype=torch.float16, device="cuda")) for _ in range(nsets)]
        res = {"MB": mb}
        for name, fn in (("library", lambda a, b: lib.sh_dma_copy(A(b), A(a), n)), ("hip_d2d", lambda a, b: b.copy_(a))):
            busy(torch, lambda: [fn(a, b) for a, b in sets], 0.1)
            ts = []
            for _ in range(3 if mb < 512 else 2):
                for a, b in sets:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn(a, b)
                    e1.record()
                    ts.append((e0, e1))
            torch.cuda.synchronize()
            us = sorted(e0.elapsed_time(e1) for e0, e1 in ts)[len(ts) // 2] * 1e3
            res[f"{name}_us"] = round(us, 2)
            res[f"{name}_GB/s"] = round(2 * n / (us * 1e-6) / 1e9, 1)
        rows.append(res)
        del sets
        torch.cuda.empty_cache()
    return {"copy_curve": rows}


def extra_configs(lib, torch, enc, x, lp, p, B: int, S: int, D: int, F: int, H: int) -> dict:
    """The other BASELINE config-4/5 measurements, outside the timed region: the 12-layer stack and batched
    attention at B=8, S=1024."""
    from softhier_mlir_amd import shops
    out = {"stack12": stack12(torch, enc, x, B, S, D, F)}
    Bl, Sl = 8, 1024
    A = shops.addr
    qkv = torch.randn((Bl * Sl, 3 * D), dtype=torch.float16, device="cuda")
    o = torch.empty((Bl * Sl, D), dtype=torch.float16, device="cuda")
    D3 = 3 * D
    def run():
        rc = lib.sh_attention_batched(A(qkv), A(qkv, D), A(qkv, 2 * D), A(o), Bl, Sl, D, H, D3, D3, D3, D,
                                      Sl * D3, Sl * D3, Sl * D3, Sl * D, 1.0 / (D // H) ** 0.5, 0)
        if rc != 0:
            raise RuntimeError(f"sh_attention_batched failed: {shops.last_error()}")
    busy(torch, run, 0.1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / 20
    aflop = 4 * Bl * H * Sl * Sl * (D // H)
    out["attention_b8_s1024"] = {"us": round(us, 2), "TFLOP/s": round(aflop / (us * 1e-6) / 1e12, 1)}
    return out


def config_table(lib, torch) -> list:
    """Every BASELINE.json config on its own (`--configs`): GPU time (median of 60 single launches with HIP events
    around each, after warm-up), parity against the oracle's restatement (which is also the timed CPU baseline:
    median of 5 runs, 3 for the long ones), and the roofline fraction: FLOP-type ops against min(MFMA peak,
    AI x HBM peak), byte-type ops against the HBM peak."""
    import numpy as np

    from oracle import refs
    from softhier_mlir_amd import data, encoder, shops
    A = shops.addr
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    host = lambda t: t.cpu().numpy()  # noqa: E731
    rows = []

    batched = {}

    def gpu_us(fn, n=60):
        """Median of n single launches with events around each; the average of n launches back to back (events
        around all of them, dispatch pipelined) is kept for the record."""
        busy(torch, fn, 0.1)
        ts = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            ts.append((e0, e1))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        batched["us"] = e0.elapsed_time(e1) * 1e3 / n
        ms = sorted(a.elapsed_time(b) for a, b in ts)
        return ms[len(ms) // 2] * 1e3

    def cpu_ms(fn, n=5):
        fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2] * 1e3

    def record(name, shape, us, flop, nbytes, got, want, cpu, exact=False, note=""):
        bad, err, _ = refs.close(got, want)
        g32, w32 = np.asarray(got, np.float32), np.asarray(want, np.float32)
        rel = float(np.max(np.abs(g32 - w32) / np.maximum(np.abs(w32), 1e-3)))
        row = {"config": name, "shape": shape, "us": round(us, 2), "us_batched": round(batched["us"], 2),
               "max_abs_err": round(err, 6), "max_rel_err": round(rel, 5), "outside_tol": bad, "cpu_ms": round(cpu, 3)}
        if exact:
            row["bit_exact"] = bool(np.array_equal(np.asarray(got).view(np.uint16), np.asarray(want).view(np.uint16)))
        ub = batched["us"]
        if flop:
            ai = flop / nbytes
            bound = min(PEAK_TFLOPS * 1e12, ai * PEAK_GBS * 1e9)
            row.update({"TFLOP/s": round(flop / (us * 1e-6) / 1e12, 2), "TFLOP/s_batched": round(flop / (ub * 1e-6) / 1e12, 2),
                        "AI": round(ai, 1), "roofline_TFLOP/s": round(bound / 1e12, 1), "frac": round(flop / (us * 1e-6) / bound, 3)})
        else:
            row.update({"GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "GB/s_batched": round(nbytes / (ub * 1e-6) / 1e9, 1),
                        "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_GBS, 3)})
        if note:
            row["note"] = note
        rows.append(row)
        print(json.dumps(row), flush=True)

    # config 1: Z[256x256] = X.W, uniform [-1, 1] from the seeded LCG
    x, w = data.uniform(256, 256, 1), data.uniform(256, 256, 2)
    X, W = dev(x), dev(w)
    Z = torch.empty((256, 256), dtype=torch.float16, device="cuda")
    us = gpu_us(lambda: lib.sh_gemm(A(X), A(W), A(Z), 256, 256, 256, 256, 256, 256, None, shops.SH_ALL))
    cpu = cpu_ms(lambda: refs.r16(refs.gemm(x, w)))
    record("1 gemm 256^3", [256, 256, 256], us, 2 * 256 ** 3, 3 * 256 * 256 * 2, host(Z), refs.r16(refs.gemm(x, w)), cpu)

    # config 2: the encoder's GEMM shapes at M = 256 with an fp32 bias U[-0.1, 0.1]; weights scaled by 1/sqrt(K)
    for name, (M, N, K, act, splits) in {"2 qkv 256x768->2304 +bias": (256, 2304, 768, 0, 1),
                                          "2 ffn_up 256x768->3072 +bias+gelu": (256, 3072, 768, shops.SH_ACT_GELU, 1),
                                          "2 ffn_down 256x3072->768 +bias split-K 4": (256, 768, 3072, 0, 4)}.items():
        x = data.uniform(M, K, 3)
        w = (data.uniform(K, N, 4).astype(np.float32) / np.sqrt(K)).astype(np.float16)
        b = (data.uniform(1, N, 5).astype(np.float32) * np.float32(0.1))
        X, W, Bb = dev(x), dev(w), dev(b)
        Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
        e = shops.epi(bias=A(Bb), bias_fmt=shops.SH_BIAS_FP32, act=act, splits=splits)
        us = gpu_us(lambda: lib.sh_gemm_ex(A(X), A(W), A(Z), M, N, K, K, N, N, None, e))

        def ref(x=x, w=w, b=b, act=act):
            z = refs.r16(refs.r16(refs.gemm(x, w)) + b)
            return refs.r16(refs.gelu(z)) if act else z
        cpu = cpu_ms(ref)
        record(name, [M, K, N], us, 2 * M * N * K, 2 * (M * K + K * N + M * N) + 4 * N, host(Z), ref(), cpu)
    x = np.full((1024, 1024), 1.0, np.float16)
    w = np.full((1024, 1024), 1.0 / 1024, np.float16)
    X, W = dev(x), dev(w)
    Z = torch.empty((1024, 1024), dtype=torch.float16, device="cuda")
    cfg = shops.cfg(256, 256, 256)
    us = gpu_us(lambda: lib.sh_gemm_mesh(A(X), A(W), A(Z), 1024, 1024, 1024, 1024, 1024, 1024, cfg))
    xs, ws = data.uniform(1024, 1024, 6), (data.uniform(1024, 1024, 7).astype(np.float32) / 32).astype(np.float16)
    Xs, Ws = dev(xs), dev(ws)
    assert lib.sh_gemm_mesh(A(Xs), A(Ws), A(Z), 1024, 1024, 1024, 1024, 1024, 1024, cfg) == 0
    cpu = cpu_ms(lambda: refs.r16(refs.gemm(xs, ws)))
    record("2 summa 1024^3 (mesh mode)", [1024, 1024, 1024], us, 2 * 1024 ** 3, 3 * 1024 * 1024 * 2, host(Z),
           refs.r16(refs.gemm(xs, ws)), cpu, note="timed on X=1, W=1/1024 (examples/gemm1024_summa.mlir:5), parity on LCG data")

    # the reference's small-M GEMM (sh_gemm_xmcast, sh_gemm.inc.c:192-344) on the SmolVLA expert / prefix shapes
    # its schedule notes list; uniform data, weights scaled by 1/sqrt(K)
    for M, N, K in [(50, 1600, 720), (50, 720, 2048), (200, 720, 960), (241, 960, 960), (200, 4096, 720)]:
        x = data.uniform(M, K, 8)
        w = (data.uniform(K, N, 9).astype(np.float32) / np.sqrt(K)).astype(np.float16)
        X, W = dev(x), dev(w)
        Z = torch.empty((M, N), dtype=torch.float16, device="cuda")
        us = gpu_us(lambda: lib.sh_gemm_xmcast(A(X), A(W), A(Z), M, N, K, K, N, N, None))
        cpu = cpu_ms(lambda: refs.r16(refs.gemm(x, w)))
        record(f"xmcast {M}x{K}->{N}", [M, K, N], us, 2 * M * N * K, 2 * (M * K + K * N + M * N), host(Z),
               refs.r16(refs.gemm(x, w)), cpu)

    # config 3: row ops at the configured shapes, values N(0, 1) unless stated
    M, D, F = 256, 768, 3072
    x = data.normal((M, D), 11)
    g, be = data.normal((1, D), 12, 1.0, 0.02), data.normal((1, D), 13, 0.0, 0.02)
    Xd, G, Be = dev(x), dev(g), dev(be)
    Y = torch.empty_like(Xd)
    us = gpu_us(lambda: lib.sh_layernorm(A(Y), A(Xd), A(G), A(Be), M, D, D, 1e-6, shops.SH_ALL))
    cpu = cpu_ms(lambda: refs.r16(refs.layernorm(x, g, be, 1e-6)))
    record("3 layernorm [256x768]", [M, D], us, 0, 2 * (2 * M * D + 2 * D), host(Y), refs.r16(refs.layernorm(x, g, be, 1e-6)), cpu)
    xs_ = data.normal((12 * 256, 256), 14, 0.0, 3.0)
    Xs_ = dev(xs_)
    Ys_ = torch.empty_like(Xs_)
    us = gpu_us(lambda: lib.sh_softmax_rows(A(Ys_), A(Xs_), 12 * 256, 256, 256, 0.125, shops.SH_ALL))
    cpu = cpu_ms(lambda: refs.r16(refs.softmax(xs_, 0.125)))
    record("3 softmax [12x256x256] scale 1/8", [12 * 256, 256], us, 0, 2 * 2 * 12 * 256 * 256, host(Ys_),
           refs.r16(refs.softmax(xs_, 0.125)), cpu)
    xg = data.normal((M, F), 15)
    Xg = dev(xg)
    Yg = torch.empty_like(Xg)
    us = gpu_us(lambda: lib.sh_gelu(A(Yg), A(Xg), M, F, F, shops.SH_ALL))
    cpu = cpu_ms(lambda: refs.r16(refs.gelu(xg)))
    record("3 gelu [256x3072]", [M, F], us, 0, 2 * 2 * M * F, host(Yg), refs.r16(refs.gelu(xg)), cpu)
    a2 = data.normal((M, D), 16)
    A2 = dev(a2)
    us = gpu_us(lambda: lib.sh_add(A(Y), A(Xd), A(A2), M, D, D, shops.SH_ALL))
    cpu = cpu_ms(lambda: refs.r16(refs.add(x, a2)))
    record("3 add [256x768]", [M, D], us, 0, 2 * 3 * M * D, host(Y), refs.r16(refs.add(x, a2)), cpu)
    us = gpu_us(lambda: lib.sh_add_bias(A(Y), A(Xd), A(Be), M, D, D, shops.SH_ALL))
    cpu = cpu_ms(lambda: refs.r16(refs.add_bias(x, be)))
    record("3 add_bias [256x768]", [M, D], us, 0, 2 * (2 * M * D + D), host(Y), refs.r16(refs.add_bias(x, be)), cpu)
    # transpose of a [768 x 256] view (ld 264) into a [256 x 768] view (ld 776): bit-exact
    src = data.normal((768, 264), 17)
    Src = dev(src)
    Dst = torch.zeros((256, 776), dtype=torch.float16, device="cuda")
    us = gpu_us(lambda: lib.sh_transpose(A(Dst), A(Src), 768, 256, 264, 776, shops.SH_ALL))
    cpu = cpu_ms(lambda: np.ascontiguousarray(src[:, :256].T))
    record("3 transpose [768x256] strided views", [768, 256], us, 0, 2 * 2 * 768 * 256, host(Dst)[:, :768],
           np.ascontiguousarray(src[:, :256].T), cpu, exact=True)

    # config 4: attention, q/k/v ~ N(0, 1) [B*S, 768], 12 heads, scale 0.125
    for Bq, Sq in ((32, 256), (8, 1024)):
        q, k, v = (data.normal((Bq * Sq, 768), s_) for s_ in (21, 22, 23))
        Q, Kt, V = dev(q), dev(k), dev(v)
        O = torch.empty_like(Q)
        us = gpu_us(lambda: lib.sh_attention_batched(A(Q), A(Kt), A(V), A(O), Bq, Sq, 768, 12, 768, 768, 768, 768,
                                                       Sq * 768, Sq * 768, Sq * 768, Sq * 768, 0.125, 0))
        cpu = cpu_ms(lambda: refs.attention_batched(q, k, v, Bq, 12, 0.125), n=3)
        record(f"4 attention B={Bq} S={Sq}", [Bq, Sq, 12, 64], us, 4 * Bq * 12 * Sq * Sq * 64, 2 * 4 * Bq * Sq * 768,
               host(O), refs.attention_batched(q, k, v, Bq, 12, 0.125), cpu)

    # config 5: the encoder layer (B = 32) and the 12-layer stack (parity on B = 2 sequences)
    Dm, Fm, Hm, Bm, Sm = 768, 3072, 12, 32, 256
    enc = encoder.Encoder(Dm, Fm, Hm)
    p = data.encoder_params(Dm, Fm, seed=100)
    lp = encoder.LayerParams.from_host(p)
    xh = data.normal((Bm * Sm, Dm), 7)
    Xe = dev(xh)
    Oe = torch.empty_like(Xe)
    us = gpu_us(lambda: enc.layer_fused(Xe, Oe, lp, Bm, Sm), n=50)
    cpu = cpu_ms(lambda: refs.encoder_layer(xh, p, Hm, B=Bm), n=3)
    fl = encoder.flops_per_layer(Bm, Sm, Dm, Fm)
    lb = sum(c["bytes"] for c in encoder.Encoder.op_costs(Bm, Sm, Dm, Fm, Hm).values())   # algorithmic bytes per layer
    record("5 encoder layer B=32 (fused sequence)", [Bm, Sm, Dm, Fm, Hm], us, fl, lb,
           host(Oe), refs.encoder_layer(xh, p, Hm, B=Bm), cpu)
    ps = [data.encoder_params(Dm, Fm, seed=100 + l) for l in range(12)]
    lps = [encoder.LayerParams.from_host(pp) for pp in ps]
    us = gpu_us(lambda: enc.forward(Xe, lps, Bm, Sm, out=Oe), n=10)
    x2 = xh[: 2 * Sm]
    X2 = dev(x2)
    O2 = torch.empty_like(X2)
    enc.forward(X2, lps, 2, Sm, out=O2)
    cpu = cpu_ms(lambda: refs.encoder_stack(x2, ps, Hm, B=2), n=3)
    record("5 encoder 12 layers B=32 (parity on 2 sequences)", [Bm, Sm, Dm, Fm, Hm, 12], us, 12 * fl,
           12 * lb, host(O2), refs.encoder_stack(x2, ps, Hm, B=2), cpu,
           note="cpu_ms is the oracle on 2 sequences")
    return rows


def library_gemm_table(lib, torch, B: int = 32, S: int = 256, D: int = 768, F: int = 3072) -> dict:
    """The layer's four GEMM shapes (M = B*S) timed three ways on the same operands: sh_gemm_ex with no epilogue,
    sh_gemm_ex with the layer's epilogue, and torch.matmul (hipBLASLt, no epilogue). Average of 50 launches back to
    back with HIP events around them, after 0.15 s of warm-up launches; the order of the three is interleaved per shape."""
    from softhier_mlir_amd import shops
    A = shops.addr
    M = B * S
    shapes = {"qkv": (3 * D, D, "bias"), "out_proj": (D, D, "bias_res"), "ffn_up": (F, D, "bias_gelu"),
              "ffn_down": (D, F, "bias_res")}
    out = {}
    for name, (N, K, epi) in shapes.items():
        g = torch.Generator(device="cuda").manual_seed(11)
        x = torch.randn((M, K), dtype=torch.float16, device="cuda", generator=g)
        w = (torch.randn((K, N), dtype=torch.float16, device="cuda", generator=g) * 0.02).contiguous()
        b = torch.zeros((1, N), dtype=torch.float16, device="cuda")
        r = torch.randn((M, N), dtype=torch.float16, device="cuda", generator=g)
        z = torch.empty((M, N), dtype=torch.float16, device="cuda")
        zt = torch.empty((M, N), dtype=torch.float16, device="cuda")
        e_plain = shops.epi()
        e_layer = shops.epi(bias=A(b), act=shops.SH_ACT_GELU if epi == "bias_gelu" else shops.SH_ACT_NONE,
                            residual=A(r) if epi == "bias_res" else 0, ldr=N if epi == "bias_res" else 0)
        runs = {
            "sh_gemm_ex_plain_us": lambda: lib.sh_gemm_ex(A(x), A(w), A(z), M, N, K, K, N, N, None, e_plain),
            "sh_gemm_ex_layer_epilogue_us": lambda: lib.sh_gemm_ex(A(x), A(w), A(z), M, N, K, K, N, N, None, e_layer),
            "torch_matmul_hipblaslt_us": lambda: torch.matmul(x, w, out=zt),
        }
        res = {}
        for key, fn in runs.items():
            busy(torch, fn, 0.15)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(50):
                fn()
            e1.record()
            torch.cuda.synchronize()
            res[key] = round(e0.elapsed_time(e1) * 1e3 / 50, 2)
        flop = 2 * M * N * K
        res["TFLOP/s_plain"] = round(flop / (res["sh_gemm_ex_plain_us"] * 1e-6) / 1e12, 1)
        res["TFLOP/s_hipblaslt"] = round(flop / (res["torch_matmul_hipblaslt_us"] * 1e-6) / 1e12, 1)
        res["shape_MNK"] = [M, N, K]
        lib.sh_gemm_ex(A(x), A(w), A(z), M, N, K, K, N, N, None, e_plain)
        torch.cuda.synchronize()
        res["max_abs_diff_plain_vs_torch"] = round(float((z.float() - zt.float()).abs().max()), 5)
        out[name] = res
    return out


def torch_layer_table(torch, enc, lp, p: dict, xh, B: int, S: int, D: int, F: int, H: int, steps: int) -> dict:
    """The bench's encoder layer (the same weights, input and the reference's op order) as a torch eager forward in
    fp16: F.layer_norm, F.linear (hipBLASLt) with the Q, K and V weights in one matrix, scaled_dot_product_attention on
    its flash backend only (no math path), F.gelu(approximate="tanh"). Both it and the library's fused layer (its
    steps chained as in the bench line) are timed over `steps` steps on the synchronised host clock after the same
    warm-up; the largest difference between the two layers' outputs for the same input."""
    import numpy as np
    import torch.nn.functional as Fn
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from softhier_mlir_amd import encoder
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    wqkv = T(np.concatenate([p["wq"], p["wk"], p["wv"]], axis=1).T)          # F.linear takes [out, in]
    bqkv = T(np.concatenate([p["bq"], p["bk"], p["bv"]], axis=1).reshape(-1))
    wo, w1, w2 = T(p["wo"].T), T(p["w1"].T), T(p["w2"].T)
    bo, b1, b2, g1, be1, g2, be2 = (T(p[k].reshape(-1)) for k in ("bo", "b1", "b2", "g1", "be1", "g2", "be2"))
    dh = D // H
    x = T(xh)

    def layer(xin):
        ln1 = Fn.layer_norm(xin, (D,), g1, be1, 1e-6)
        qkv = Fn.linear(ln1, wqkv, bqkv)
        q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(B, S, H, dh).transpose(1, 2) for i in range(3))
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            o = Fn.scaled_dot_product_attention(q, k, v, scale=1.0 / dh ** 0.5)
        h = xin + Fn.linear(o.transpose(1, 2).reshape(B * S, D), wo, bo)
        f = Fn.gelu(Fn.linear(Fn.layer_norm(h, (D,), g2, be2, 1e-6), w1, b1), approximate="tanh")
        return h + Fn.linear(f, w2, b2)

    ours = torch.empty_like(x)
    enc.layer_fused(x, ours, lp, B, S, x_parts=False)
    theirs = layer(x)
    torch.cuda.synchronize()
    diff = float((ours.float() - theirs.float()).abs().max())
    bufs, n = (x.clone(), torch.empty_like(x)), [0]

    def lib_step():
        i = n[0]
        n[0] += 1
        enc.layer_fused(bufs[i % 2], bufs[(i + 1) % 2], lp, B, S, x_parts=i > 0)
    res = {}
    for name, fn in (("library_fused", lib_step), ("torch_eager", lambda: layer(x))):
        busy(torch, fn, 0.3)
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        res[name] = {"ms_per_step": round(ms, 4),
                     "TFLOP/s": round(encoder.flops_per_layer(B, S, D, F) / (ms * 1e-3) / 1e12, 1)}
    res["max_abs_diff_library_vs_torch"] = round(diff, 5)
    res["config"] = {"batch": B, "seq_len": S, "d_model": D, "ffn": F, "heads": H, "steps": steps}
    return res


def torch_rowops_table(lib, torch, B: int = 32, S: int = 256, D: int = 768, F: int = 3072, H: int = 12) -> dict:
    """The row ops at the batched shapes through the library and through torch's own kernels for the same operation
    (torch.nn.functional.layer_norm, torch.softmax, gelu(approximate="tanh"), torch.add, the broadcast bias add,
    a transposed view copied into a contiguous output), cold: buffer sets rotated over >= 512 MiB as in the bench's
    row-op section, after the warm-up; the median of single launches with HIP events around each and the average of
    all sets back to back, and the largest difference between the two outputs of one set. Softmax runs unscaled
    (torch's kernel has no scale)."""
    from softhier_mlir_amd import shops
    A = shops.addr
    M = B * S
    ops = {"layernorm": (M, D), "softmax": (H * M, S), "gelu": (M, F), "add": (M, D), "add_bias": (M, D), "transpose": (M, D)}
    out = {}
    for name, (r, c) in ops.items():
        nbytes = 2 * 3 * r * c if name == "add" else 2 * 2 * r * c
        nsets = max(2, int((512 << 20) // nbytes) + 1)
        g = torch.Generator(device="cuda").manual_seed(5)
        gamma = torch.rand((c,), dtype=torch.float16, device="cuda", generator=g) + 0.5
        beta = torch.rand((c,), dtype=torch.float16, device="cuda", generator=g) - 0.5
        sets = []
        for _ in range(nsets):
            x = torch.randn((r, c), dtype=torch.float16, device="cuda", generator=g)
            y = torch.empty((c, r) if name == "transpose" else (r, c), dtype=torch.float16, device="cuda")
            yt = torch.empty_like(y)
            b = torch.randn((r, c), dtype=torch.float16, device="cuda", generator=g) if name == "add" else None
            sets.append((x, y, yt, b))

        def run_lib(x, y, yt, b):
            if name == "layernorm":
                lib.sh_layernorm(A(y), A(x), A(gamma), A(beta), r, c, c, 1e-6, shops.SH_ALL)
            elif name == "softmax":
                lib.sh_softmax_rows(A(y), A(x), r, c, c, 1.0, shops.SH_ALL)
            elif name == "gelu":
                lib.sh_gelu(A(y), A(x), r, c, c, shops.SH_ALL)
            elif name == "add":
                lib.sh_add(A(y), A(x), A(b), r, c, c, shops.SH_ALL)
            elif name == "add_bias":
                lib.sh_add_bias(A(y), A(x), A(beta), r, c, c, shops.SH_ALL)
            else:
                lib.sh_transpose(A(y), A(x), r, c, c, r, shops.SH_ALL)

        def run_torch(x, y, yt, b):
            if name == "layernorm":
                torch.nn.functional.layer_norm(x, (c,), gamma, beta, 1e-6)   # (allocates its output)
            elif name == "softmax":
                torch.softmax(x, dim=-1, out=yt)
            elif name == "gelu":
                torch.nn.functional.gelu(x, approximate="tanh")       # (torch allocates its output: no out= form)
            elif name == "add":
                torch.add(x, b, out=yt)
            elif name == "add_bias":
                torch.add(x, beta, out=yt)
            else:
                yt.copy_(x.t())

        def timed(fn):
            busy(torch, lambda: [fn(*st) for st in sets], 0.15)
            ts = []
            for _ in range(3):
                for st in sets:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn(*st)
                    e1.record()
                    ts.append((e0, e1))
            torch.cuda.synchronize()
            ms = sorted(a.elapsed_time(b) for a, b in ts)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for st in sets:
                fn(*st)
            e1.record()
            torch.cuda.synchronize()
            return ms[len(ms) // 2] * 1e3, e0.elapsed_time(e1) * 1e3 / len(sets)

        lu, lb = timed(run_lib)
        tu, tb = timed(run_torch)
        x, y, yt, b = sets[0]
        run_lib(x, y, yt, b)
        ref = {"layernorm": lambda: torch.nn.functional.layer_norm(x, (c,), gamma, beta, 1e-6),
               "softmax": lambda: torch.softmax(x, dim=-1), "gelu": lambda: torch.nn.functional.gelu(x, approximate="tanh"),
               "add": lambda: x + b, "add_bias": lambda: x + beta, "transpose": lambda: x.t().contiguous()}[name]()
        torch.cuda.synchronize()
        out[name] = {"shape": [r, c], "bytes": nbytes, "library_us": round(lu, 2), "library_us_batched": round(lb, 2),
                     "torch_us": round(tu, 2), "torch_us_batched": round(tb, 2),
                     "library_GB/s_batched": round(nbytes / (lb * 1e-6) / 1e9, 1),
                     "torch_GB/s_batched": round(nbytes / (tb * 1e-6) / 1e9, 1),
                     "max_abs_diff": round(float((y.float() - ref.float()).abs().max()), 5)}
        del sets
        torch.cuda.empty_cache()
    return out


def torch_sdpa_table(lib, torch) -> dict:
    """Batched attention through sh_attention_batched next to torch.nn.functional.scaled_dot_product_attention on
    the same fp16 operands ([B, H, S, 64] contiguous for torch), restricted to its flash and memory-efficient
    backends (a backend that is not available raises; no fallback to the math path). Average of 50 launches back to
    back with HIP events around them, after the warm-up; the largest difference between the two outputs."""
    from softhier_mlir_amd import shops
    from torch.nn.attention import SDPBackend, sdpa_kernel
    A = shops.addr
    out = {}
    for B, S in ((32, 256), (8, 1024)):
        H, dh = 12, 64
        D = H * dh
        g = torch.Generator(device="cuda").manual_seed(3)
        q = torch.randn((B, S, D), dtype=torch.float16, device="cuda", generator=g)
        k, v = torch.randn_like(q), torch.randn_like(q)
        o = torch.empty_like(q)

        def lib_call():
            rc = lib.sh_attention_batched(A(q), A(k), A(v), A(o), B, S, D, H, D, D, D, D, S * D, S * D, S * D, S * D,
                                          0.125, 0)
            if rc != 0:
                raise RuntimeError(f"sh_attention_batched failed: {shops.last_error()}")
        qh, kh, vh = (t.view(B, S, H, dh).transpose(1, 2).contiguous() for t in (q, k, v))

        def timed(fn, n=50):
            busy(torch, fn, 0.1)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(n):
                fn()
            e1.record()
            torch.cuda.synchronize()
            return round(e0.elapsed_time(e1) * 1e3 / n, 2)
        res = {"sh_attention_batched_us": timed(lib_call)}
        flop = 4 * B * H * S * S * dh
        res["TFLOP/s_library"] = round(flop / (res["sh_attention_batched_us"] * 1e-6) / 1e12, 1)
        for name, backend in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
            try:
                with sdpa_kernel([backend]):
                    sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, scale=0.125)  # noqa: E731
                    got = sdpa()
                    torch.cuda.synchronize()
                    res[f"torch_sdpa_{name}_us"] = timed(sdpa)
                    res[f"max_abs_diff_{name}_vs_library"] = round(
                        float((got.transpose(1, 2).reshape(B, S, D).float() - o.float()).abs().max()), 5)
            except RuntimeError as e:
                res[f"torch_sdpa_{name}"] = f"unavailable: {str(e)[:120]}"
        out[f"B{B}_S{S}"] = res
    return out


def cpu_baseline(B: int, S: int, D: int, F: int, H: int, p: dict, x) -> dict:
    """The oracle's numpy restatement of one encoder layer, timed on this host's cores (median of 5)."""
    import numpy as np

    from oracle import refs
    threads = None
    try:
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=None)
    except Exception:
        pass
    Bs = min(B, 8)                                   # bounded sample: 8 of the 32 sequences
    xs = x[: Bs * S]
    refs.encoder_layer(xs, p, H, B=Bs)               # warm-up
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        refs.encoder_layer(xs, p, H, B=Bs)
        ts.append(time.perf_counter() - t0)
    med = sorted(ts)[2]
    from softhier_mlir_amd.encoder import flops_per_layer
    value = flops_per_layer(Bs, S, D, F) / med / 1e12
    return {"value": round(value, 4), "unit": "TFLOP/s", "cores": threads or os.cpu_count(), "kind": "port",
            "sample": f"numpy fp32 oracle of one layer on {Bs} of the {B} sequences (S={S}), median of 5 runs "
                      f"({med:.3f} s each); host cpu_count={os.cpu_count()} affinity={len(os.sched_getaffinity(0))}"}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build (the encoder path would "
              f"shard by sequence, one GPU per group of sequences, with no exchange)", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from softhier_mlir_amd import data, encoder, shops

    lib = shops.load()
    lib.sh_init()
    if args.configs:
        config_table(lib, torch)
        return 0
    if args.library_gemm:
        print(json.dumps({"library_gemm": library_gemm_table(lib, torch, args.batch, args.seq)}), flush=True)
        return 0
    if args.torch_rowops:
        print(json.dumps({"torch_rowops": torch_rowops_table(lib, torch)}), flush=True)
        return 0
    if args.torch_sdpa:
        print(json.dumps({"torch_sdpa": torch_sdpa_table(lib, torch)}), flush=True)
        return 0
    if args.copy_curve:
        print(json.dumps(copy_curve(lib, torch)), flush=True)
        return 0
    B, S, D, F, H = args.batch, args.seq, 768, 3072, 12
    p = data.encoder_params(D, F, seed=100)
    xh = data.normal((B * S, D), 7)
    x = torch.from_numpy(xh).cuda()
    out = torch.empty_like(x)
    enc = encoder.Encoder(D, F, H)
    enc.row_partials = not args.row_stats
    if args.stack:
        print(json.dumps({"stack12": stack12(torch, enc, x, B, S, D, F, reps=args.steps, warmup=args.warmup)}), flush=True)
        return 0
    lp = encoder.LayerParams.from_host(p)
    if args.torch_layer:
        print(json.dumps({"torch_layer": torch_layer_table(torch, enc, lp, p, xh, B, S, D, F, H, args.steps)}), flush=True)
        return 0
    if args.sequence == "fused":
        # one layer of the 12-layer stack as it runs there: each step reads the rows the previous step stored, and
        # the row partials its FFN-down wrote (five launches); the first step starts with sh_row_stats
        bufs, nstep = (x, out), [0]

        def step(*_):
            i = nstep[0]
            nstep[0] += 1
            enc.layer_fused(bufs[i % 2], bufs[(i + 1) % 2], lp, B, S, x_parts=i > 0)
    else:
        def step(*_):
            enc.layer_reference(x, out, lp, B, S)

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.float16, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step(x, out, lp, B, S)
    busy(torch, step, 0.3)

    events: dict = {}

    class Tap:
        """HIP events (torch's current stream = the legacy null stream the library launches on) around one op.
        The events are created ahead (`pool`), so recording them costs the host little and the host keeps ahead
        of the GPU: an event pair then brackets the kernel, not an idle gap before it."""
        only = None
        pool: list = []

        def __init__(self, name):
            self.name = name
            self.on = Tap.only is None or name == Tap.only

        def __enter__(self):
            if self.on:
                if not Tap.pool:
                    Tap.pool = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                                for _ in range(256)]
                self.e0, self.e1 = Tap.pool.pop()
                self.e0.record()

        def __exit__(self, *exc):
            if self.on:
                self.e1.record()
                events.setdefault(self.name, []).append((self.e0, self.e1))
            return False

    def avg_us(evs):
        return sum(a.elapsed_time(b) for a, b in evs) / len(evs) * 1e3

    costs = encoder.Encoder.op_costs(B, S, D, F, H)
    breakdown = {}
    if args.sequence == "fused":
        # untimed breakdown pass: events around every op, to name the dominant kernel
        enc.tap = Tap
        for _ in range(max(5, min(args.steps, 20))):
            step(x, out, lp, B, S)
        torch.cuda.synchronize()
        for name, evs in events.items():
            us = avg_us(evs)
            c = costs[name]
            entry = {"us": round(us, 2)}
            if c["flop"]:
                entry["TFLOP/s"] = round(c["flop"] / (us * 1e-6) / 1e12, 1)
                entry["mfma_frac"] = round(c["flop"] / (us * 1e-6) / 1e12 / PEAK_TFLOPS, 3)
            entry["GB/s"] = round(c["bytes"] / (us * 1e-6) / 1e9, 1)
            breakdown[name] = entry
        events.clear()
        Tap.only = max(breakdown, key=lambda k: breakdown[k]["us"])   # the dominant op (its launches are timed below)

    # timed region: K steps, each one replay of the captured layer graph (or the eager op sequence)
    graph = None
    enc.tap = None
    eager_ms = None
    if args.sequence == "fused" and args.graph:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step(x, out, lp, B, S)
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        graph = enc.capture(x, out, lp, B, S)
        for _ in range(args.warmup):
            graph.replay()
        busy(torch, graph.replay, 0.2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step(x, out, lp, B, S)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    flop = encoder.flops_per_layer(B, S, D, F)
    value = flop / (elapsed / args.steps) / 1e12

    # the dominant op's average launch duration: its library call of the steady-state step (same kernel, same
    # operands) launched K times back to back between one HIP event pair on the library stream, so the pair's
    # own dispatch overhead (a few us per pair, more under a kernel tracer) is spread over K launches
    dom_us = None
    if Tap.only is not None and args.sequence == "fused":
        plan = {nm: (fn, a) for nm, fn, a, _ in enc._fused_plan(bufs[0], bufs[1], lp, B, S, True)}
        fn, a = plan[Tap.only]
        fn(*a)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            fn(*a)
        e1.record()
        torch.cuda.synchronize()
        dom_us = e0.elapsed_time(e1) * 1e3 / args.steps

    roofline = None
    if dom_us is not None:
        dom = Tap.only
        c = costs[dom]
        us = dom_us
        if c["flop"]:
            ach = c["flop"] / (us * 1e-6) / 1e12
            roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_TFLOPS, 4), "traffic": counted_traffic(dom),
                        "algorithmic_flop_per_launch": c["flop"], "algorithmic_bytes_per_launch": c["bytes"],
                        "avg_launch_us": round(us, 2)}
            tr = traced_avg_us(dom)
            if tr is not None:          # the committed kernel trace's average for the same op, and its fraction
                roofline.update({"trace_kernel": tr[0], "trace_avg_launch_us": tr[1],
                                 "trace_frac": round(c["flop"] / (tr[1] * 1e-6) / 1e12 / PEAK_TFLOPS, 4),
                                 "trace_figures_us": tr[2],
                                 "trace_source": "profiles/encoder_layer_b32_s256_kernel_trace.md"})
        else:
            ach = c["bytes"] / (us * 1e-6) / 1e9
            roofline = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / PEAK_GBS, 4), "traffic": counted_traffic(dom),
                        "algorithmic_bytes_per_launch": c["bytes"], "avg_launch_us": round(us, 2)}

    extra = {} if args.no_extra else extra_configs(lib, torch, enc, x, lp, p, B, S, D, F, H)
    rowops = None if args.no_rowops else rowops_bandwidth(lib, torch, B, S, D, F, H)
    rowops_large = None if args.no_rowops else rowops_bandwidth(lib, torch, B, S, D, F, H, reps=2, scale=16)
    cpu = None if args.no_cpu else cpu_baseline(B, S, D, F, H, p, xh)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) input)",
        "config": {"workload": f"SigLIP-B encoder layer forward, {args.sequence} op sequence"
                               + (", HIP graph replay" if graph is not None else ", eager launches"), "global_batch": B,
                   "seq_len": S, "d_model": D, "ffn": F, "heads": H, "layers": 1, "parallelism": "single GPU"},
        "mfma_frac_of_peak": round(value / PEAK_TFLOPS, 4),
        "eager_ms_per_step": round(eager_ms, 4) if eager_ms is not None else None,
        "roofline": roofline, "breakdown": breakdown, **extra, "rowops": rowops, "rowops_x16_rows": rowops_large,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
