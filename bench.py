#!/usr/bin/env python3
"""Benchmark of the batch-1 decode hot path on one MI355X.

One step = one pass over the OLMo-2-1B-shaped decode-step linear set at M = 1 in bf16 (byteprof_amd/decode_set.py):
16 layers x (q, k, v, o 2048 -> 2048; gate, up 2048 -> 8192; down 8192 -> 2048) + the LM head 2048 -> 100352,
113 linears, every weight distinct (2.56 GB, ten times the 256 MB Infinity Cache), all operands resident in HBM
before the timed region. The reference's set semantics: every linear reads its own seeded unit-RMS input, as in
byteprof's set benchmark, where each linear is an independent skinny call (tools/skinny_bench.py:45-71). The step
runs as one grouped launch (csrc/skinny_group.hip): one grid over the row blocks of all 113 linears, every output
bitwise equal to its own skinny_mm call.

Printed (one JSON line): the step's aggregate HBM throughput (algorithmic bytes = weights + activations + outputs,
each once: 2,560,237,568 B per step) in GB/s, us per set and % of the 8 TB/s peak; the roofline of the grouped
kernel (the only kernel of the step): algorithmic bytes per launch over the average launch duration, from HIP
events on the launch stream over the timed steps, and the HBM traffic per launch from the committed rocprofv3
counter summary (profiles/skinny_group_kernel_decode_set.md); the CPU baseline (torch F.linear, the reference's
CPU path for these linears, on the host cores); and secondary figures: the same set in one launch of the
persistent set kernel (csrc/linear_set.hip), independent and as a dependent decode chain (each stage reads the
renormalised output it depends on), the 113-launch HIP graph of skinny kernels (the reference's execution model),
the int8 set (fp16 scales) the same ways, the fused mLSTM block, the bf16 verify-width sweep (M = 1..16, VALU /
matrix-core kernels), and the graph-captured greedy decode loop of the OLMo-2-1B-shaped model (us per token, bf16
and int8).

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


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


PROFILE = ROOT / "profiles" / "skinny_dot_kernel_decode_set.md"
GROUP_PROFILE = ROOT / "profiles" / "skinny_group_kernel_decode_set.md"


def per_shape(ops, kind: str, m: int) -> dict:
    """Per (N, K): launches per set, us per launch in a graph of all the set's launches of that shape, algorithmic
    bytes, and the kernel instantiation it uses."""
    from byteprof_amd import decode_set as D
    from byteprof_amd.quant.accounting import Linear, call_bytes

    groups: dict[tuple[int, int], list] = {}
    for op in ops:
        groups.setdefault((op.n, op.k), []).append(op)
    scheme = None if kind == "bf16" else "int8_wo"
    res = {}
    for (n, k), group in groups.items():
        g = D.capture(group)
        D.time_replays(g, 2, 1)
        reps = max(1, 64 // len(group))
        us = statistics.median(D.time_replays(g, reps, 5)) * 1000.0 / len(group)
        nbytes = call_bytes(Linear(n, k), scheme, m)
        res[f"{n}x{k}"] = {"launches": len(group), "us": us, "bytes": int(nbytes), "gbs": nbytes / us / 1e3,
                           "kernel": D.kernel_key(kind, n, k, m)}
        del g
    return res


def profiled_traffic(path: Path = PROFILE) -> dict[tuple[str, str], float]:
    """(kernel, 'NxK' or workload tag) -> HBM bytes per launch from a committed counter summary ('traffic:'
    lines)."""
    out = {}
    if path.exists():
        for line in path.read_text().splitlines():
            if line.startswith("traffic: "):
                kernel, shape, nbytes = line[len("traffic: "):].rsplit(" ", 2)
                out[(kernel, shape)] = float(nbytes)
    return out


def roofline(shapes: dict) -> dict:
    """The kernel instantiation with the largest total time per step: algorithmic bytes of its launches over their
    average duration; traffic from the profile when it covers every shape this instantiation serves."""
    by_kernel: dict[str, list] = {}
    for key, s in shapes.items():
        by_kernel.setdefault(s["kernel"], []).append((key, s))
    name, items = max(by_kernel.items(), key=lambda kv: sum(s["us"] * s["launches"] for _, s in kv[1]))
    launches = sum(s["launches"] for _, s in items)
    t = sum(s["us"] * s["launches"] for _, s in items)
    b = sum(s["bytes"] * s["launches"] for _, s in items)
    achieved = b / t / 1e3
    prof = profiled_traffic()
    traffic = None
    if all((name, k) in prof for k, _ in items):
        traffic = sum(prof[(name, k)] * s["launches"] for k, s in items) / launches
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "kernel": name,
            "shapes": [k for k, _ in items], "launches_per_step": launches,
            "avg_us_per_launch": t / launches, "avg_bytes_per_launch": b / launches}


def cpu_baseline(ops, budget_s: float = 20.0) -> dict:
    """torch F.linear on the host cores over the decode-step set (bf16 weights copied to host memory), the
    reference's CPU path for these linears (byteprof/optim/skinny_linear.py:67-68). Bounded: passes run while they
    fit in the budget (at most 5); the median pass is reported."""
    import torch
    import torch.nn.functional as F

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():  # the host's CPU share for this GPU, when it is set
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(cores)
    host = [(op.args[0].cpu(), op.x.cpu()) for op in ops]
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
    cpu = "unknown"
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
    from a graph of 64 launches (dispatch gap included)."""
    import torch

    from byteprof_amd import decode_set as D
    from byteprof_amd.optim import draft_fused

    g = torch.Generator(device=device).manual_seed(0)
    t, nh, dq, dv = 16, 4, 256, 256
    r = lambda *s: torch.randn(*s, generator=g, device=device)  # noqa: E731
    q, k, v = (r(t, nh, d).to(torch.bfloat16) for d in (dq, dq, dv))
    i, f = r(t, nh, 1), r(t, nh, 1) + 3.0
    state = (r(1, nh, dq, dv) * 0.1, r(1, nh, dq) * 0.1, r(1, nh, 1))
    h = torch.empty(t, nh, dv, dtype=torch.bfloat16, device=device)
    ns, ms = torch.empty(nh, dq, device=device), torch.empty(nh, device=device)
    gr = D.capture([lambda: draft_fused.multistep_fw(state, q, k, v, i, f, h, ns, ms, eps=1e-6)] * 64)
    us = statistics.median(D.time_replays(gr, 10, 5)) * 1000.0 / 64
    nbytes = 2 * (4 * (nh * dq * dv + nh * dq + nh)) + t * (2 * (2 * nh * dq + nh * dv) + 2 * 4 * nh + 2 * nh * dv)
    return {"config": "NH=4, DQ=DV=256, T=16, bf16 io, fp32 gates/state", "us_per_block": us,
            "us_per_step": us / t, "bytes": nbytes, "gbs": nbytes / us / 1e3}


def time_launches(run, steps: int, warmup: int) -> tuple[float, float]:
    """(ms per launch from HIP events on the launch stream, ms per launch by the host clock) over `steps`
    back-to-back launches of `run` (one launch each, on torch's current stream) after `warmup` untimed ones,
    synchronised on both sides."""
    import torch

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        run()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return ev0.elapsed_time(ev1) / steps, wall_ms


def time_set(lset, steps: int, warmup: int) -> tuple[float, float]:
    """time_launches of the persistent set kernel, checking that no launch gave up waiting."""
    out = time_launches(lset.run, steps, warmup)
    if lset.timed_out():
        raise RuntimeError("a set launch gave up waiting for another workgroup: its results are invalid")
    return out


def _figures(ev_ms: float, wall_ms: float, nbytes: int) -> dict:
    ms = max(ev_ms, wall_ms)
    return {"us_per_set": ms * 1e3, "gbs": nbytes / ms / 1e6, "pct_of_hbm_peak": nbytes / ms / 1e6 / HBM_PEAK_GBS
            * 100}


def set_figures(lset, nbytes: int, steps: int) -> dict:
    return {**_figures(*time_set(lset, steps, max(2, steps // 10)), nbytes), "stages": len(lset.stages)}


def group_roofline(group, ev_ms: float, nbytes: int, tag: str) -> dict:
    """Roofline of the grouped kernel: algorithmic bytes per launch over the HIP-event launch time, traffic per
    launch from the committed counter summary."""
    kernel = f"skinny_group_kernel<{0 if group.kind == 'bf16' else 1}, {group.rows}, {group.waves}>"
    achieved = nbytes / (ev_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic(GROUP_PROFILE).get((kernel, tag)), "kernel": kernel, "launches_per_step": 1,
            "avg_us_per_launch": ev_ms * 1e3, "bytes_per_launch": nbytes, "workgroups": group.blocks}


def per_launch_graph(ops, kind: str, nbytes: int) -> dict:
    """The same linears as a HIP graph of one skinny launch each (the reference's execution model)."""
    from byteprof_amd import decode_set as D

    g = D.capture(ops)
    D.time_replays(g, 5, 1)
    ms = statistics.median(D.time_replays(g, 20, 5))
    del g
    out = {"launches": len(ops), "us_per_set": ms * 1e3, "gbs": nbytes / ms / 1e6,
           "pct_of_hbm_peak": nbytes / ms / 1e6 / HBM_PEAK_GBS * 100}
    if kind == "bf16":
        shapes = per_shape(ops, kind, 1)
        out["kernels"] = shapes
        out["roofline"] = roofline(shapes)
        out["empty_launch_us"] = D.dispatch_gap_us()
    return out


def sweep(device) -> dict:
    """The verify-width sweep: us per skinny_mm call for M in {1, 2, 4, 8, 16} x K in {2048, 8192} x N in {2048,
    8192, 100352} (bf16), each cell over a ring of >= 1 GiB of distinct weights in one HIP graph (weights streamed
    from HBM), with the kernel family skinny_mm routes the row count to."""
    import torch

    from byteprof_amd import decode_set as D
    from byteprof_amd.optim import skinny as S

    out = {}
    for n in (2048, 8192, 100352):
        for k in (2048, 8192):
            per = 2 * n * k
            ring = [(torch.randn(n, k, device=device) * 0.02).to(torch.bfloat16) for _ in range(max(2, (1 << 30) // per))]
            cell = {}
            for m in (1, 2, 4, 8, 16):
                x = torch.randn(m, k, device=device).to(torch.bfloat16)
                y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
                g = D.capture([lambda w=w: S.skinny_mm(x, w, out=y) for w in ring])
                us = statistics.median(D.time_replays(g, 2, 5)) * 1000.0 / len(ring)
                del g
                fam = "mf"
                cell[str(m)] = {"us": round(us, 2), "gbs": round((per + 2 * m * (n + k)) / us / 1e3), "kernel": fam}
            out[f"{n}x{k}"] = cell
            del ring
            torch.cuda.empty_cache()
    return out


def draft_figures(dec, prompt, ref, new_tokens: int) -> dict:
    """The drafting loop (byteprof_amd/optim/olmo_draft.py) on the same decoder: the captured verify round's GPU
    time for K drafts (K + 1 rows; replays back to back, events), and the loop's time per token with the oracle
    drafter (the recorded greedy continuation: every draft accepted, the upper bound of a drafter), K up to 8. The
    recorded continuation is the drafting loop's own: its rows from 5 on use the matrix-core linears, which can
    part from the one-token loop at a near tie, so the graph loop's tokens are re-recorded through the drafting
    loop until they repeat (at most 3 passes)."""
    import torch

    from byteprof_amd.optim import olmo_draft as OD

    key = tuple(prompt[0].tolist())
    truth = {key: ref[0, prompt.shape[1]:].tolist()}
    stats = OD.Stats()
    gen, st = OD.make_generate_draft(dec, {"kind": "oracle", "truth": truth}, stats)
    out = gen(prompt, max_new_tokens=4)  # captures the rounds' graphs
    same = 1
    for _ in range(3):
        out = gen(prompt, max_new_tokens=1 + new_tokens)
        toks = out[0, prompt.shape[1]:].tolist()
        if toks == truth[key]:
            break
        same = 0
        truth[key] = toks
    stats.__init__()
    t0 = time.perf_counter()
    gen(prompt, max_new_tokens=1)
    t1 = time.perf_counter()
    out = gen(prompt, max_new_tokens=1 + new_tokens)
    t2 = time.perf_counter()
    rounds = {}
    for k, g in st["graphs"].items():
        dec.v_pos.fill_(prompt.shape[1])
        g.replay()
        torch.cuda.synchronize()
        dec.v_pos.fill_(prompt.shape[1])
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        reps = 20
        ev[0].record()
        for _ in range(reps):
            g.replay()
        ev[1].record()
        ev[1].synchronize()
        rounds[str(k + 1)] = ev[0].elapsed_time(ev[1]) / reps * 1e3
    per_token = ((t2 - t1) - (t1 - t0)) / new_tokens * 1e6
    return {"us_per_round_by_rows": rounds, "oracle_drafter_us_per_token": per_token,
            "oracle_drafter_tokens_per_s": 1e6 / per_token, "same_tokens_as_graph_loop": same,
            "rounds": stats.rounds, "tokens": stats.emitted,
            "note": "oracle drafter: every draft accepted (the recorded continuation of this loop); rounds of 9 rows"}


def decode_loop(device, new_tokens: int = 128) -> dict:
    """The graph-captured greedy decode loop (byteprof_amd/optim/olmo.py) on the OLMo-2-1B shape with synthetic
    weights: per kind, the GPU time of one captured decode step (replays timed with events), the loop's time per
    token (one replay + one pinned read + one sync; a generate of 1 + N tokens minus one of 1, over N) and the
    eager loop's, with the weight bytes a step streams."""
    import torch

    from byteprof_amd.optim import olmo as OG

    cfg = OG.OLMO2_1B
    prompt = torch.tensor([[11, 2027, 5, 99999, 42, 3, 3, 1000]])
    out = {"model": "OLMo-2-1B shape (16 x 2048, FFN 8192, 16 heads, vocab 100352), synthetic weights",
           "prompt_tokens": prompt.shape[1], "new_tokens": new_tokens}
    for kind in ("bf16", "int8"):
        dec = OG.OlmoDecoder(cfg, OG.random_weights(cfg, device, seed=4), kind)
        out["launches_per_step"] = dec.launches_per_step
        graph = OG.make_generate_graph(dec)
        graph(prompt, max_new_tokens=4)  # captures the step
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graph(prompt, max_new_tokens=1)
        t1 = time.perf_counter()
        ref = graph(prompt, max_new_tokens=1 + new_tokens)
        t2 = time.perf_counter()
        loop_us = ((t2 - t1) - (t1 - t0)) / new_tokens * 1e6
        eager = OG.make_generate(dec)
        e0 = time.perf_counter()
        eager(prompt, max_new_tokens=1)
        e1 = time.perf_counter()
        eager(prompt, max_new_tokens=1 + 32)
        e2 = time.perf_counter()
        eager_us = ((e2 - e1) - (e1 - e0)) / 32 * 1e6
        # the captured step alone: replays back to back, timed on the GPU
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        reps = 50
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            dec.step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            dec.step()
        dec.pos.zero_()
        g.replay()
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(reps):
            g.replay()
        ev[1].record()
        ev[1].synchronize()
        step_us = ev[0].elapsed_time(ev[1]) / reps * 1e3
        nb = dec.weight_bytes()
        out[kind] = {"us_per_token_loop": loop_us, "us_per_step_graph": step_us, "us_per_token_eager": eager_us,
                     "weight_bytes_per_step": nb, "weight_gbs_graph_step": nb / step_us / 1e3,
                     "tokens_per_s_loop": 1e6 / loop_us, "draft": draft_figures(dec, prompt, ref, new_tokens)}
        del dec, graph, eager, g
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="skip the secondary figures")
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
    from byteprof_amd import decode_set as D

    _lib.lib()
    log("[bench] building the bf16 decode-step set (2.56 GB of weights)")
    weights = D.make_weights("bf16", device, seed=0)
    ops = D.build("bf16", 1, device, seed=0, weights=weights)
    group = D.group_of(ops)
    nbytes = D.chain_bytes("bf16")
    log(f"[bench] warm-up {a.warmup}, timing {a.steps} steps")
    ev_ms, wall_ms = time_launches(group.run, a.steps, a.warmup)
    ms = max(ev_ms, wall_ms)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] {ms * 1e3:.1f} us per set, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")

    result = {
        "metric": METRIC, "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0, 0.02^2) bf16 weights, unit-RMS N(0,1) activations)",
        "config": {"workload": ("OLMo-2-1B-shaped decode-step linear set at M=1, bf16: 16 x (q,k,v,o 2048->2048; "
                                "gate,up 2048->8192; down 8192->2048) + LM head 2048->100352, 113 linears with "
                                "their own inputs, one grouped launch"),
                   "M": 1, "linears": len(D.shapes()), "bytes_per_step": nbytes, "us_per_set": ms * 1e3,
                   "pct_of_hbm_peak": gbs / HBM_PEAK_GBS * 100, "event_ms": ev_ms, "wall_ms": wall_ms},
        "roofline": group_roofline(group, ev_ms, nbytes, "group-bf16"),
    }
    if not a.no_extras:
        log("[bench] persistent set kernel, independent and dependent")
        ind = D.build_chain("bf16", device, dependent=False, weights=weights)
        dep = D.build_chain("bf16", device, dependent=True, weights=weights)
        result["persistent_set"] = {"independent": set_figures(ind.lset, nbytes, 100),
                                    "dependent_chain": set_figures(dep.lset, nbytes, 50)}
        del ind, dep
        log("[bench] 113-launch graph")
        result["per_launch_graph"] = per_launch_graph(ops, "bf16", nbytes)
        log("[bench] int8 set")
        w8 = D.make_weights("int8", device, seed=0)
        nb8 = D.chain_bytes("int8")
        ops8 = D.build("int8", 1, device, seed=0, weights=w8)
        group8 = D.group_of(ops8)
        # 1000 untimed launches first (~0.2 s): the int8 kernel's conversion work makes it sensitive to the core
        # clock, which drops while the host builds the int8 weights and takes that long to come back up
        ev8, wall8 = time_launches(group8.run, 100, 1000)
        grp8 = {**_figures(ev8, wall8, nb8), "roofline": group_roofline(group8, ev8, nb8, "group-int8")}
        ind8 = D.build_chain("int8", device, dependent=False, weights=w8)
        i8 = set_figures(ind8.lset, nb8, 100)
        del ind8
        dep8 = D.build_chain("int8", device, dependent=True, weights=w8)
        d8 = set_figures(dep8.lset, nb8, 50)
        del dep8
        g8 = per_launch_graph(ops8, "int8", nb8)
        del ops8, group8
        result["int8_set"] = {"bytes_per_step": nb8, "scales": "fp16 per output row", "grouped": grp8,
                              "persistent_set": {"independent": i8, "dependent_chain": d8}, "per_launch_graph": g8,
                              "bf16_over_int8_time": ms * 1e3 / grp8["us_per_set"],
                              "bf16_over_int8_time_dependent": result["persistent_set"]["dependent_chain"]
                              ["us_per_set"] / d8["us_per_set"]}
        del w8
        torch.cuda.empty_cache()
        log("[bench] mLSTM block")
        result["mlstm"] = mlstm_block(device)
        log("[bench] verify-width sweep")
        result["sweep_bf16"] = sweep(device)
        log("[bench] decode loop")
        result["decode_loop"] = decode_loop(device)
    if not a.no_cpu:
        log("[bench] CPU baseline")
        result["cpu_baseline"] = cpu_baseline(ops)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
