#!/usr/bin/env python3
"""Benchmark of the batch-1 decode hot path on one MI355X.

One step = one replay of a HIP graph holding the OLMo-2-1B-shaped decode-step linear set at M = 1 in bf16:
16 layers x (q, k, v, o 2048 -> 2048; gate, up 2048 -> 8192; down 8192 -> 2048) + the LM head 2048 -> 100352,
113 skinny launches in decode order, every weight distinct (2.56 GB, ten times the 256 MB Infinity Cache, so
nothing stays cached between replays). Weights ~ N(0, 0.02^2), each linear's input ~ N(0, 1) renormalised to unit
RMS, all resident in HBM before the timed region.

Printed (rank 0, one JSON line): the set's aggregate HBM throughput (algorithmic bytes = weights + activations +
outputs, each once, 2,560,237,568 B per step) in GB/s and as a fraction of the 8 TB/s peak; us per set; the
roofline of the dominant kernel (average launch duration measured with HIP events on the launch stream over a
graph of all its launches); the CPU baseline (torch F.linear, the reference's CPU path for these linears, on the
host cores, bounded sample); and secondary figures (per-shape launch times, the int8 set, the fused mLSTM block).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extras]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "skinny GEMM achieved HBM GB/s (% peak) at M=1; us per decode-step linear set"
LAYERS = 16
HIDDEN, FFN, VOCAB = 2048, 8192, 100352
LAYER_LINEARS = [("q", HIDDEN, HIDDEN), ("k", HIDDEN, HIDDEN), ("v", HIDDEN, HIDDEN), ("o", HIDDEN, HIDDEN),
                 ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN), ("down", HIDDEN, FFN)]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def decode_set() -> list[tuple[str, int, int]]:
    """(name, N, K) of the 113 linears in decode order."""
    out = [(f"l{layer}.{name}", n, k) for layer in range(LAYERS) for name, n, k in LAYER_LINEARS]
    out.append(("lm_head", VOCAB, HIDDEN))
    return out


def unit_rms(x):
    import torch

    xf = x.float()
    return (xf / xf.pow(2).mean(dim=-1, keepdim=True).sqrt()).to(torch.bfloat16)


def build_operands(kind: str, m: int, device, seed: int = 0):
    """Per linear: (name, n, k, weight args, x, y). kind 'bf16' or 'int8' (fp16 per-row scales)."""
    import torch

    from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8

    g = torch.Generator(device=device).manual_seed(seed)
    ops = []
    for name, n, k in decode_set():
        w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        if kind == "bf16":
            args = (w,)
        else:
            q, s = quantize_rowwise_int8(w, torch.float16)
            args = (q, s)
            del w
        x = unit_rms(torch.randn(m, k, generator=g, device=device))
        y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
        ops.append((name, n, k, args, x, y))
    return ops


def algorithmic_bytes(ops, kind: str, m: int) -> int:
    from byteprof_amd.quant.accounting import Linear, call_bytes

    scheme = None if kind == "bf16" else "int8_wo"
    return int(sum(call_bytes(Linear(n, k), scheme, m) for _, n, k, _, _, _ in ops))


def capture(calls):
    """Capture the callables in one HIP graph (after a warm-up on a side stream)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    torch.cuda.synchronize()
    return g


def time_replays(g, replays: int, trials: int) -> list[float]:
    """ms per replay for each trial (HIP events on the current stream, which the replays run on)."""
    import torch

    out = []
    for _ in range(trials):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(replays):
            g.replay()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) / replays)
    return out


def launch_calls(ops):
    from byteprof_amd.optim import skinny as S

    return [(lambda a=args, x=x, y=y: S.skinny_mm(x, *a, out=y)) for _, _, _, args, x, y in ops]


def per_shape_launch_times(ops, kind: str, m: int) -> dict:
    """Average launch duration per (N, K) shape: one graph of all the set's launches of that shape."""
    from byteprof_amd.optim import skinny as S
    from byteprof_amd.quant.accounting import Linear, call_bytes

    shapes: dict[tuple[int, int], list] = {}
    for op in ops:
        shapes.setdefault((op[1], op[2]), []).append(op)
    scheme = None if kind == "bf16" else "int8_wo"
    res = {}
    for (n, k), group in shapes.items():
        g = capture(launch_calls(group))
        reps = max(1, 64 // len(group))
        time_replays(g, 2, 1)
        us = statistics.median(time_replays(g, reps, 5)) * 1000.0 / len(group)
        nbytes = call_bytes(Linear(n, k), scheme, m)
        rows, waves, split = S._resolve(kind, n, k, S._bm(m), None)
        res[f"{n}x{k}"] = {"launches": len(group), "us": us, "bytes": int(nbytes), "gbs": nbytes / us / 1e3,
                           "cfg": {"rows": rows, "waves": waves, "split": split}}
        del g
    return res


def cpu_baseline(ops, budget_s: float = 20.0) -> dict:
    """torch F.linear on the host cores over the decode-step set (bf16 weights copied to host memory), the
    reference's CPU path for these linears (byteprof/optim/skinny_linear.py:67-68). Bounded: the first full pass
    is timed; further passes run while they fit in the budget; the median pass is reported."""
    import platform

    import torch
    import torch.nn.functional as F

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():  # the host's CPU share for this GPU, when it is set
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(cores)
    host = [(args[0].cpu(), x.cpu()) for _, _, _, args, x, _ in ops]
    nbytes = sum(w.numel() * w.element_size() + 2 * (x.numel() + w.shape[0]) for w, x in host)
    for w, x in host[:4]:
        F.linear(x, w)
    passes = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        for w, x in host:
            F.linear(x, w)
        passes.append(time.perf_counter() - t0)
        if len(passes) >= 5 or time.perf_counter() + passes[-1] > t_end:
            break
    sec = statistics.median(passes)
    cpu = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": nbytes / sec / 1e9, "unit": "GB/s", "cores": cores, "kind": "reference",
            "sample": (f"torch.nn.functional.linear, bf16, M=1, over the full 113-linear decode-step set "
                       f"({len(passes)} passes, median {sec * 1e3:.1f} ms per set) on {cpu}"),
            "ms_per_set": sec * 1e3}


def mlstm_block(device) -> dict:
    """The fused mLSTM multistep: NH = 4, DQ = DV = 256, T = 16, bf16 q/k/v, fp32 gates and state; us per launch
    from a graph of 64 launches."""
    import torch

    from byteprof_amd.optim import draft_fused

    g = torch.Generator(device=device).manual_seed(0)
    t, nh, dq, dv = 16, 4, 256, 256
    r = lambda *s: torch.randn(*s, generator=g, device=device)  # noqa: E731
    q, k, v = (r(t, nh, d).to(torch.bfloat16) for d in (dq, dq, dv))
    i, f = r(t, nh, 1), r(t, nh, 1) + 3.0
    state = (r(1, nh, dq, dv) * 0.1, r(1, nh, dq) * 0.1, r(1, nh, 1))
    h = torch.empty(t, nh, dv, dtype=torch.bfloat16, device=device)
    ns, ms = torch.empty(nh, dq, device=device), torch.empty(nh, device=device)
    calls = [lambda: draft_fused.multistep_fw(state, q, k, v, i, f, h, ns, ms, eps=1e-6)] * 64
    gr = capture(calls)
    us = statistics.median(time_replays(gr, 10, 5)) * 1000.0 / 64
    nbytes = 2 * (4 * (nh * dq * dv + nh * dq + nh)) + t * (2 * (2 * nh * dq + nh * dv) + 2 * 4 * nh + 2 * nh * dv)
    return {"config": "NH=4, DQ=DV=256, T=16, bf16 io, fp32 gates/state", "us_per_block": us,
            "us_per_step": us / t, "bytes": nbytes, "gbs": nbytes / us / 1e3}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="skip the per-shape, int8 and mLSTM figures")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the decode hot path is single-GPU, batch 1 "
              f"(asked for --gpus {a.gpus}, WORLD_SIZE {world})", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    from byteprof_amd import _lib

    _lib.lib()

    log("[bench] building the bf16 decode-step set (2.56 GB of weights)")
    ops = build_operands("bf16", 1, device, seed=0)
    nbytes = algorithmic_bytes(ops, "bf16", 1)
    g = capture(launch_calls(ops))
    log("[bench] warm-up")
    for _ in range(a.warmup):
        g.replay()
    torch.cuda.synchronize()
    log(f"[bench] timing {a.steps} steps")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(a.steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / a.steps
    ev_ms = ev0.elapsed_time(ev1) / a.steps
    ms = max(wall_ms, ev_ms)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] {ms * 1e3:.1f} us per set, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")

    result = {
        "metric": METRIC, "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0, 0.02^2) bf16 weights, unit-RMS N(0,1) activations)",
        "config": {"workload": ("OLMo-2-1B-shaped decode-step linear set at M=1, bf16: 16 x (q,k,v,o 2048->2048; "
                                "gate,up 2048->8192; down 8192->2048) + LM head 2048->100352, 113 skinny launches "
                                "in one HIP graph"),
                   "M": 1, "linears": len(ops), "bytes_per_step": nbytes, "us_per_set": ms * 1e3,
                   "pct_of_hbm_peak": gbs / HBM_PEAK_GBS * 100, "event_ms": ev_ms, "wall_ms": wall_ms},
    }

    shapes = per_shape_launch_times(ops, "bf16", 1)
    dom_key = max(shapes, key=lambda s: shapes[s]["us"] * shapes[s]["launches"])
    dom = shapes[dom_key]
    result["roofline"] = {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": dom["gbs"] / HBM_PEAK_GBS, "traffic": None,
                          "kernel": f"skinny_dot_kernel bf16 {dom_key} (N x K), M=1",
                          "us_per_launch": dom["us"], "bytes_per_launch": dom["bytes"]}
    if not a.no_extras:
        result["kernels"] = shapes
        del g
        ops8 = None
        try:
            log("[bench] int8 set")
            ops8 = build_operands("int8", 1, device, seed=0)
            nb8 = algorithmic_bytes(ops8, "int8", 1)
            g8 = capture(launch_calls(ops8))
            time_replays(g8, 5, 1)
            ms8 = statistics.median(time_replays(g8, 20, 5))
            result["int8_set"] = {"us_per_set": ms8 * 1e3, "bytes_per_step": nb8, "gbs": nb8 / (ms8 * 1e-3) / 1e9,
                                  "bf16_over_int8_time": ms / ms8, "scales": "fp16 per output row"}
            del g8
        finally:
            del ops8
        log("[bench] mLSTM block")
        result["mlstm"] = mlstm_block(device)
    if not a.no_cpu:
        log("[bench] CPU baseline")
        result["cpu_baseline"] = cpu_baseline(ops)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
