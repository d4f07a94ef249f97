"""Benchmark of the softhier-ops hot path on one MI355X: the SigLIP-B encoder layer (
B=32, S=256, D=768, 12 heads, FFN 3072, fp16, weights N(0, 0.02), biases zero, x ~ N(0, 1), seeded).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--sequence fused|reference] [--graph] [--no-cpu] [--no-rowops]

A step is one forward pass of the layer over the batch through libshops.so (inputs resident in HBM), its calls
launched one by one; `--graph` records the fused layer's seven calls once into a HIP graph and times replays of
it instead (the same kernels every step; on MI355X this measured no faster: the gaps between kernels are not
host launch time). Prints ONE JSON line with the whole-job TFLOP/s, the roofline of the dominant kernel (HIP events around its
launches, on the library stream = the legacy null stream torch also uses), the per-op breakdown, the row-op HBM
bandwidths at the batched shapes (cold: rotating buffer sets of >= 512 MiB; each next to a plain device copy of
the same bytes, the practical ceiling at that size) and the numpy CPU baseline (the oracle's restatement, timed
on this host).
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
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the 12-layer stack and the S=1024 attention measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 3 plain device copies of 512 MiB (a known-size kernel for scaling HBM counters)")
    return ap.parse_args()


def counted_traffic(op: str):
    """HBM bytes per launch of `op` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by a
    known-size copy; profiles/*hbm_counters.md), or None when no summary covers the op."""
    for f in sorted((ROOT / "profiles").glob("*hbm_counters.md")):
        for line in f.read_text().splitlines():
            if line.startswith(f"traffic_bytes_per_launch {op}:"):
                return int(line.split(":")[1])
    return None


def rowops_bandwidth(lib, torch, B: int, S: int, D: int, F: int, H: int, reps: int = 3) -> dict:
    """Row ops at the batched shapes, cold: buffer sets rotated so that >= 512 MiB is touched between reuses
    (MI355X Infinity Cache = 256 MiB). Algorithmic bytes: each input read once, the output written once."""
    from softhier_mlir_amd import shops
    A = shops.addr
    M = B * S
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
            y.view(-1).copy_(x.view(-1))

        def timed(fn):
            """(median us of single launches with events around each, us per launch of all sets back to back)"""
            for st in sets:
                fn(*st)
            torch.cuda.synchronize()
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


def extra_configs(lib, torch, enc, x, lp, p, B: int, S: int, D: int, F: int, H: int) -> dict:
    """The other BASELINE config-4/5 measurements, outside the timed region: the 12-layer stack (layer l reads
    layer l-1's output; weights of layer l seeded 100 + l) and batched attention at B=8, S=1024."""
    from softhier_mlir_amd import data, encoder, shops
    out = {}
    layers = [encoder.LayerParams.from_host(data.encoder_params(D, F, seed=100 + l)) for l in range(12)]
    y = torch.empty_like(x)
    enc.forward(x, layers, B, S, out=y)                 # warm-up (buffers, tile choices)
    torch.cuda.synchronize()
    reps = 5
    t0 = time.perf_counter()
    for _ in range(reps):
        enc.forward(x, layers, B, S, out=y)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    flop = 12 * encoder.flops_per_layer(B, S, D, F)
    out["stack12"] = {"layers": 12, "ms_per_forward": round(ms, 3), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 1)}
    del layers, y
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
    for _ in range(3):
        run()
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
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build (the path shards by "
              f"sequence across GPUs; see DESIGN.md)", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from softhier_mlir_amd import data, encoder, shops

    lib = shops.load()
    lib.sh_init()
    B, S, D, F, H = args.batch, args.seq, 768, 3072, 12
    p = data.encoder_params(D, F, seed=100)
    xh = data.normal((B * S, D), 7)
    x = torch.from_numpy(xh).cuda()
    out = torch.empty_like(x)
    enc = encoder.Encoder(D, F, H)
    lp = encoder.LayerParams.from_host(p)
    step = enc.layer_fused if args.sequence == "fused" else enc.layer_reference

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.float16, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step(x, out, lp, B, S)
    torch.cuda.synchronize()

    events: dict = {}

    class Tap:
        """HIP events (torch's current stream = the legacy null stream the library launches on) around one op."""
        only = None

        def __init__(self, name):
            self.name = name
            self.on = Tap.only is None or name == Tap.only

        def __enter__(self):
            if self.on:
                self.e0 = torch.cuda.Event(enable_timing=True)
                self.e1 = torch.cuda.Event(enable_timing=True)
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
        Tap.only = max(breakdown, key=lambda k: breakdown[k]["us"])   # only the dominant op is timed below

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

    # the dominant op's launches, timed with HIP events in K eager steps right after (same kernels, same shapes)
    if Tap.only is not None:
        enc.tap = Tap
        for _ in range(args.steps):
            step(x, out, lp, B, S)
        torch.cuda.synchronize()
        enc.tap = None

    roofline = None
    if Tap.only is not None:
        dom = Tap.only
        c = costs[dom]
        us = avg_us(events[dom])
        if c["flop"]:
            ach = c["flop"] / (us * 1e-6) / 1e12
            roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_TFLOPS, 4), "traffic": counted_traffic(dom),
                        "algorithmic_flop_per_launch": c["flop"], "algorithmic_bytes_per_launch": c["bytes"],
                        "avg_launch_us": round(us, 2)}
        else:
            ach = c["bytes"] / (us * 1e-6) / 1e9
            roofline = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / PEAK_GBS, 4), "traffic": counted_traffic(dom),
                        "algorithmic_bytes_per_launch": c["bytes"], "avg_launch_us": round(us, 2)}

    extra = {} if args.no_extra else extra_configs(lib, torch, enc, x, lp, p, B, S, D, F, H)
    rowops = None if args.no_rowops else rowops_bandwidth(lib, torch, B, S, D, F, H)
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
        "roofline": roofline, "breakdown": breakdown, **extra, "rowops": rowops, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
