#!/usr/bin/env python3
"""Benchmark of the batch-1 decode hot path on one MI355X.

One step = one pass over the OLMo-2-1B-shaped decode-step linear set at M = 1 in bf16 (byteprof_amd/decode_set.py):
16 layers x (q, k, v, o 2048 -> 2048; gate, up 2048 -> 8192; down 8192 -> 2048) + the LM head 2048 -> 100352,
113 linears, every weight distinct (2.56 GB, ten times the 256 MB Infinity Cache), all operands resident in HBM
before the timed region.

`value` is the sequential figure: the set as the 65 stream-ordered skinny launches a decode step makes (q|k|v and
gate|up each one launch over adjacent weight rows; o, down and the head one each), in one HIP graph, each launch
starting after the one before it has finished, every stage reading its own seeded unit-RMS input. The reference's
execution model is the same sequence with one skinny call per linear (byteprof/optim/olmo.py:164-215; its set
benchmark times those calls, tools/skinny_bench.py:45-71): that 113-launch graph is reported beside it.

Printed (one JSON line): GB/s of the step (algorithmic bytes = weights + activations + outputs, each once:
2,560,237,568 B per step), us per set and % of the 8 TB/s peak; `roofline` for the dominant (kernel instantiation,
shape) pair, the one with the largest time per step (its launches' algorithmic bytes over their average duration
from HIP events, HBM traffic per launch from the committed rocprofv3 counter summary), with `shapes` giving the same
figures for every shape of the set; `copy_ceiling`: a 256 MiB device copy (read + write counted), the ceiling the
reference reports (tools/skinny_bench.py:74-81); config.floor_us_stream_ordered: 65 empty launches plus the set's
bytes at the one-launch grid's read rate; `cpu_baseline`: torch F.linear over the set on the host cores (the
reference's CPU path); secondary figures:
  - graph_113: the 113 linears as one skinny launch each (the reference's sequence);
  - one_launch_set: the same 113 independent linears as one grid (csrc/skinny_chain.hip), with its own roofline;
  - dependent: the set with real data dependencies (each stage reads the unit-RMS renormalisation of the output it
    depends on in a decode step) as 65 stream-ordered skinny launches (the renormalisation inside each launch), as
    one launch of the chain kernel (in-kernel hand-off) and as 65 launches of the chain kernel (those two give
    bitwise equal outputs, checked here);
  - int8_set: the int8 weight-only set (fp16 scales) in the same execution models (its stage graph with a
    per-shape roofline), and as 113-launch graphs at M = 4 and 16; bf16 / int8 time ratios;
  - int4: the group-128 int4 kernel on the set's shapes;
  - c1: one 8192 x 2048 linear at M = 1 (GPU, and F.linear on the CPU);
  - mlstm: the fused 16-step mLSTM block;
  - sweep_bf16 / sweep_int8: the verify widths M in {1, 2, 4, 8, 16} x K {2048, 8192} x N {2048, 8192, 100352};
  - decode_loop: the graph-captured greedy decode loop of the OLMo-2-1B shape (bf16, int8, int4) and its drafting loop;
  - cpu_legs: on the host cores, fp32 F.linear over the full 113-linear set, int8 dequantize-then-F.linear over
    the full set, the 8192 x 2048 linear alone, and the mLSTM block as a torch fp32 step loop.
Every timed leg is warmed by time (WARM_S seconds of its own launches) first.

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
WARM_S = 0.5
SET_PROFILE = ROOT / "profiles" / "skinny_mf_kernel_decode_set.md"
CHAIN_PROFILE = ROOT / "profiles" / "chain_kernel_decode_set.md"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _sync():
    import torch

    torch.cuda.synchronize()


def warm(fn, seconds: float = WARM_S) -> int:
    """Runs fn until `seconds` have passed (synchronising each time); returns the runs."""
    t_end = time.perf_counter() + seconds
    runs = 0
    while True:
        fn()
        _sync()
        runs += 1
        if time.perf_counter() >= t_end:
            return runs


def time_runs(fn, steps: int, warmup: int = 0, warm_s: float = WARM_S) -> tuple[float, float]:
    """(ms per run from HIP events on torch's current stream, ms per run by the host clock) over `steps`
    back-to-back runs of fn, after warm-up by time (and at least `warmup` runs); synchronised on both sides."""
    import torch

    warm(fn, warm_s)
    for _ in range(warmup):
        fn()
    _sync()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        fn()
    ev1.record()
    _sync()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return ev0.elapsed_time(ev1) / steps, wall_ms


def figures(ms: float, nbytes: int) -> dict:
    gbs = nbytes / ms / 1e6
    return {"us_per_set": ms * 1e3, "gbs": gbs, "pct_of_hbm_peak": gbs / HBM_PEAK_GBS * 100}


def profiled_traffic(path: Path) -> dict[tuple[str, str], float]:
    """(kernel, 'NxK' or workload tag) -> HBM bytes per launch from a committed counter summary ('traffic:'
    lines)."""
    out = {}
    if path.exists():
        for line in path.read_text().splitlines():
            if line.startswith("traffic: "):
                kernel, shape, nbytes = line[len("traffic: "):].rsplit(" ", 2)
                out[(kernel, shape)] = float(nbytes)
    return out


def graph_of(calls):
    from byteprof_amd import decode_set as D

    return D.capture(calls)


def per_shape(ops, kind: str, m: int) -> dict:
    """Per (N, K): launches per set, us per launch in a graph of all the set's launches of that shape (warmed by
    time), algorithmic bytes, and the kernel instantiation it uses."""
    from byteprof_amd import decode_set as D
    from byteprof_amd.quant.accounting import Linear, call_bytes

    groups: dict[tuple[int, int], list] = {}
    for op in ops:
        groups.setdefault((op.n, op.k), []).append(op)
    scheme = None if kind == "bf16" else "int8_wo"
    res = {}
    for (n, k), group in groups.items():
        g = graph_of(group)
        reps = max(1, 64 // len(group))
        ev_ms, _ = time_runs(g.replay, reps, warm_s=0.1)
        us = ev_ms * 1e3 / len(group)
        nbytes = call_bytes(Linear(n, k), scheme, m)
        res[f"{n}x{k}"] = {"launches": len(group), "us": us, "bytes": int(nbytes), "gbs": nbytes / us / 1e3,
                           "kernel": D.kernel_key(kind, n, k, m)}
        del g
    return res


def roofline_of_graph(shapes: dict) -> dict:
    """The dominant (kernel instantiation, shape) pair, the one with the largest time per step: its algorithmic
    bytes per launch over its average launch duration (HIP events over a graph of the set's launches of that shape),
    HBM traffic per launch from the committed counter summary; `shapes` lists the same figures for every shape of
    the set (one entry each)."""
    prof = profiled_traffic(SET_PROFILE)
    entries = []
    for key, s in shapes.items():
        e = {"shape": key, "kernel": s["kernel"], "launches_per_step": s["launches"], "us_per_launch": s["us"],
             "us_per_step": s["us"] * s["launches"], "bytes_per_launch": s["bytes"], "achieved": s["gbs"],
             "frac": s["gbs"] / HBM_PEAK_GBS, "traffic": prof.get((s["kernel"], key))}
        entries.append(e)
    entries.sort(key=lambda e: -e["us_per_step"])
    top = entries[0]
    return {"bound": "hbm", "achieved": top["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": top["frac"],
            "traffic": top["traffic"], "kernel": top["kernel"], "shape": top["shape"],
            "launches_per_step": top["launches_per_step"], "avg_us_per_launch": top["us_per_launch"],
            "bytes_per_launch": top["bytes_per_launch"], "shapes": entries}


def copy_ceiling(device, mib: int = 256) -> dict:
    """GB/s of a large device-to-device copy (read + write counted), timed as a HIP graph of copies: the streaming
    ceiling the reference reports beside its skinny figures (tools/skinny_bench.py:74-81)."""
    import torch

    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=device)
    b = torch.empty_like(a)
    g = graph_of([lambda: b.copy_(a)] * 10)
    ev_ms, _ = time_runs(g.replay, 7, warm_s=0.2)
    del g, a, b
    us = ev_ms * 1e3 / 10
    gbs = 2 * n / us / 1e3
    return {"gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "us_per_copy": us, "bytes_moved": 2 * n,
            "method": f"torch copy_ of {mib} MiB (read + write counted), graph of 10 copies, HIP events"}


def chain_roofline(lc, ev_ms: float, nbytes: int, tag: str) -> dict:
    """Roofline of a one-launch set: algorithmic bytes per launch over the HIP-event launch time; traffic per launch
    from the committed counter summary."""
    kernel = f"chain_kernel<{0 if lc.kind == 'bf16' else 1}, {lc.waves}>"
    achieved = nbytes / (ev_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic(CHAIN_PROFILE).get((kernel, tag)), "kernel": kernel, "launches_per_step": 1,
            "avg_us_per_launch": ev_ms * 1e3, "bytes_per_launch": nbytes, "workgroups": lc.total_wgs}


def one_launch(kind: str, weights, nbytes: int, device, waves: int, tag: str) -> dict:
    """The 113 independent linears as one grid (rows per workgroup sized per linear), with its roofline."""
    from byteprof_amd import decode_set as D

    ch = D.build_chain(kind, device, weights=weights, dependent=False, waves=waves)
    ev_ms, wall_ms = time_runs(ch.lset.run, 100)
    out = {**figures(max(ev_ms, wall_ms), nbytes), "waves": waves,
           "roofline": chain_roofline(ch.lset, ev_ms, nbytes, tag)}
    del ch
    return out


def dependent_figures(kind: str, weights, nbytes: int, device) -> dict:
    """The set with a decode step's data dependencies: 65 stream-ordered skinny launches (renormalisation inside
    each launch); one launch of the chain kernel (in-kernel hand-off between stages) and 65 stream-ordered launches
    of it, whose outputs must be equal bit for bit."""
    import torch

    from byteprof_amd import decode_set as D

    ch = D.build_chain(kind, device, weights=weights, dependent=True)
    gs = graph_of(D.stage_graph_calls(ch))
    evs, _ = time_runs(gs.replay, 50)
    del gs
    skinny_stages = {**figures(evs, nbytes), "launches": len(ch.stages)}
    ev_ms, wall_ms = time_runs(ch.lset.run, 50)
    if ch.lset.timed_out():
        raise RuntimeError("a dependent launch gave up waiting: its results are invalid")
    one = {**figures(max(ev_ms, wall_ms), nbytes), "launches": 2, "stages": len(ch.stages)}
    ref = [st.out.clone() for st in ch.stages]
    stages = D.stage_launches(ch)
    g = graph_of([lc.run for lc in stages])
    ev2, _ = time_runs(g.replay, 50)
    g.replay()
    _sync()
    same = all(torch.equal(a, st.out) for a, st in zip(ref, ch.stages))
    out = {"skinny_stage_graph": skinny_stages, "chain_one_launch": one,
           "chain_stage_graph": {**figures(ev2, nbytes), "launches": len(stages)}, "chain_outputs_equal": bool(same)}
    del g, stages, ch, ref
    return out


def graph_set(kind: str, weights, m: int, device, seed: int = 0) -> dict:
    """The 113 linears at M rows as stream-ordered skinny_mm launches in one HIP graph."""
    from byteprof_amd import decode_set as D
    from byteprof_amd.quant.accounting import Linear, call_bytes

    ops = D.build(kind, m, device, seed=seed, weights=weights)
    scheme = None if kind == "bf16" else "int8_wo"
    nbytes = int(sum(call_bytes(Linear(op.n, op.k), scheme, m) for op in ops))
    g = graph_of(ops)
    ev_ms, _ = time_runs(g.replay, 20)
    del g, ops
    return {**figures(ev_ms, nbytes), "launches": len(D.shapes()), "M": m, "bytes": nbytes}


def int4_figures(device) -> dict:
    """The group-128 int4 kernel at M = 1 on the set's shapes, the weights packed with the tuned tile rows: us per
    call over a ring of distinct weights, bytes stored (codes + bf16 scales + fp16 zeros + activations + outputs)."""
    import torch

    from byteprof_amd.optim import skinny as S

    out = {}
    for n, k in ((2048, 2048), (8192, 2048), (2048, 8192), (100352, 2048)):
        w = (torch.randn(n, k, device=device) * 0.02).to(torch.bfloat16)
        packed, sc, z = S.quantize_int4(w, S.int4_tile_rows(n, k))
        del w
        per = packed.numel() + sc.numel() * 2 + z.numel() * 2
        ring = [(packed, sc, z)] + [(packed.clone(), sc.clone(), z.clone()) for _ in range(max(1, (1 << 29) // per) - 1)]
        x = torch.randn(1, k, device=device).to(torch.bfloat16)
        y = torch.empty(1, n, dtype=torch.bfloat16, device=device)
        g = graph_of([lambda a=a: S.skinny_mm(x, *a, out=y) for a in ring])
        ev_ms, _ = time_runs(g.replay, 5, warm_s=0.2)
        us = ev_ms * 1e3 / len(ring)
        nbytes = per + 2 * (n + k)
        out[f"{n}x{k}"] = {"us": us, "gbs_stored_bytes": nbytes / us / 1e3, "bytes": nbytes,
                           "tile_rows": int(packed.shape[2])}
        del g, ring, packed, sc, z
        torch.cuda.empty_cache()
    return out


def c1_figures(device) -> dict:
    """One linear at M = 1: y = x W^T, x [1, 2048], W [8192, 2048] bf16 ~ N(0, 0.02^2), over a ring of
    distinct weights (streamed from HBM); the CPU F.linear figure is in cpu_legs."""
    import torch

    from byteprof_amd.optim import skinny as S

    n, k = 8192, 2048
    ring = [(torch.randn(n, k, device=device) * 0.02).to(torch.bfloat16) for _ in range(64)]
    x = torch.randn(1, k, device=device).to(torch.bfloat16)
    y = torch.empty(1, n, dtype=torch.bfloat16, device=device)
    g = graph_of([lambda w=w: S.skinny_mm(x, w, out=y) for w in ring])
    ev_ms, _ = time_runs(g.replay, 10, warm_s=0.2)
    us = ev_ms * 1e3 / len(ring)
    nbytes = 2 * n * k + 2 * (n + k)
    del g, ring
    return {"us": us, "gbs": nbytes / us / 1e3, "pct_of_hbm_peak": nbytes / us / 1e3 / HBM_PEAK_GBS * 100,
            "floor_us": nbytes / HBM_PEAK_GBS / 1e3}


def mlstm_block(device) -> dict:
    """The fused mLSTM multistep: NH = 4, DQ = DV = 256, T = 16, bf16 q/k/v, fp32 gates and state; us per launch
    from a graph of 64 launches (dispatch gap included)."""
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
    gr = graph_of([lambda: draft_fused.multistep_fw(state, q, k, v, i, f, h, ns, ms, eps=1e-6)] * 64)
    ev_ms, _ = time_runs(gr.replay, 10, warm_s=0.2)
    us = ev_ms * 1e3 / 64
    nbytes = 2 * (4 * (nh * dq * dv + nh * dq + nh)) + t * (2 * (2 * nh * dq + nh * dv) + 2 * 4 * nh + 2 * nh * dv)
    return {"config": "NH=4, DQ=DV=256, T=16, bf16 io, fp32 gates/state", "us_per_block": us,
            "us_per_step": us / t, "bytes": nbytes, "gbs": nbytes / us / 1e3}


def sweep(device, kind: str) -> dict:
    """Verify widths: us per skinny_mm call for M in {1, 2, 4, 8, 16} x K in {2048, 8192} x N in {2048, 8192,
    100352}, each cell over a ring of >= 1 GiB of distinct weights in one HIP graph (weights streamed from HBM)."""
    import torch

    from byteprof_amd.optim import skinny as S
    from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8

    out = {}
    for n in (2048, 8192, 100352):
        for k in (2048, 8192):
            per = (2 if kind == "bf16" else 1) * n * k
            ring = []
            for _ in range(max(2, (1 << 30) // per)):
                w = (torch.randn(n, k, device=device) * 0.02).to(torch.bfloat16)
                ring.append((w,) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16))
                del w
            cell = {}
            for m in (1, 2, 4, 8, 16):
                x = torch.randn(m, k, device=device).to(torch.bfloat16)
                y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
                g = graph_of([lambda a=a: S.skinny_mm(x, *a, out=y) for a in ring])
                ev_ms, _ = time_runs(g.replay, 3, warm_s=0.1)
                us = ev_ms * 1e3 / len(ring)
                del g
                nb = per + (2 * n if kind == "int8" else 0) + 2 * m * (n + k)
                cell[str(m)] = {"us": round(us, 2), "gbs": round(nb / us / 1e3)}
            cell["m16_over_m1"] = round(cell["16"]["us"] / cell["1"]["us"], 3)
            out[f"{n}x{k}"] = cell
            del ring
            torch.cuda.empty_cache()
    return out


def draft_figures(dec, prompt, ref, new_tokens: int) -> dict:
    """The drafting loop (byteprof_amd/optim/olmo_draft.py) on the same decoder: the captured verify round's GPU
    time for K drafts (K + 1 rows; replays back to back, events), and the loop's time per token with the oracle
    drafter (the graph loop's recorded greedy continuation: every draft accepted, the upper bound of a drafter), K
    up to 8. same_tokens_as_graph_loop: the drafting loop emits exactly the one-token loop's tokens."""
    import torch

    from byteprof_amd.optim import olmo_draft as OD

    key = tuple(prompt[0].tolist())
    truth = {key: ref[0, prompt.shape[1]:].tolist()}
    stats = OD.Stats()
    gen, st = OD.make_generate_draft(dec, {"kind": "oracle", "truth": truth}, stats)
    gen(prompt, max_new_tokens=4)  # captures the rounds' graphs
    out = gen(prompt, max_new_tokens=1 + new_tokens)
    same = int(out[0, prompt.shape[1]:].tolist() == truth[key])
    stats.__init__()
    t0 = time.perf_counter()
    gen(prompt, max_new_tokens=1)
    t1 = time.perf_counter()
    gen(prompt, max_new_tokens=1 + new_tokens)
    t2 = time.perf_counter()
    rounds = {}
    for k, g in st["graphs"].items():
        dec.v_pos.fill_(prompt.shape[1])
        g.replay()
        _sync()
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
            "note": "oracle drafter: every draft accepted (the graph loop's continuation); rounds of up to 9 rows"}


def decode_loop(device, new_tokens: int = 128) -> dict:
    """The graph-captured greedy decode loop (byteprof_amd/optim/olmo.py) on the OLMo-2-1B shape with synthetic
    weights: per kind, the GPU time of one captured decode step (replays timed with events), the loop's time per
    token (two-step graph replays kept one ahead of the host; a generate of 1 + N tokens minus one of 1, over N) and the
    eager loop's, with the weight bytes a step streams; the drafting rounds of each."""
    import torch

    from byteprof_amd.optim import olmo as OG

    cfg = OG.OLMO2_1B
    prompt = torch.tensor([[11, 2027, 5, 99999, 42, 3, 3, 1000]])
    out = {"model": "OLMo-2-1B shape (16 x 2048, FFN 8192, 16 heads, vocab 100352), synthetic weights",
           "prompt_tokens": prompt.shape[1], "new_tokens": new_tokens}
    for kind in ("bf16", "int8", "int4"):
        dec = OG.OlmoDecoder(cfg, OG.random_weights(cfg, device, seed=4), kind)
        if kind != "int4":
            out["launches_per_step"] = dec.launches_per_step
        graph = OG.make_generate_graph(dec)
        graph(prompt, max_new_tokens=4)  # captures the step
        warm(lambda: graph(prompt, max_new_tokens=8), 0.3)
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
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            dec.step()
        torch.cuda.current_stream().wait_stream(s)
        _sync()
        with torch.cuda.graph(g):
            dec.step()
        dec.pos.zero_()
        count = [0]

        def replay():  # positions 0..127 over and over (the cache rows a 128-token continuation attends to)
            count[0] += 1
            if count[0] % 128 == 0:
                dec.pos.zero_()
            g.replay()

        ev_ms, _ = time_runs(replay, 50, warm_s=0.2)
        step_us = ev_ms * 1e3
        nb = dec.weight_bytes()
        out[kind] = {"us_per_token_loop": loop_us, "us_per_step_graph": step_us, "us_per_token_eager": eager_us,
                     "weight_bytes_per_step": nb, "weight_gbs_graph_step": nb / step_us / 1e3,
                     "tokens_per_s_loop": 1e6 / loop_us}
        if kind == "int4":
            out[kind]["launches_per_step"] = dec.launches_per_step
        out[kind]["draft"] = draft_figures(dec, prompt, ref, new_tokens)
        del dec, graph, eager, g
        torch.cuda.empty_cache()
    return out


def _cores() -> int:
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():  # the host's CPU share for this GPU, when it is set
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    return cores


def _cpu_name() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_passes(fn, budget_s: float, max_passes: int = 5) -> tuple[float, int]:
    fn()  # first touch
    passes = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        fn()
        passes.append(time.perf_counter() - t0)
        if len(passes) >= max_passes or time.perf_counter() + passes[-1] > t_end:
            return statistics.median(passes), len(passes)


def cpu_baseline(weights, budget_s: float = 15.0) -> dict:
    """torch F.linear on the host cores over the bf16 decode-step set (weights copied to host memory), the
    reference's CPU path for these linears (byteprof/optim/skinny_linear.py:67-68). Bounded: passes run while they
    fit in the budget (at most 5); the median pass is reported."""
    import torch
    import torch.nn.functional as F

    from byteprof_amd import decode_set as D

    cores = _cores()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    host = [(weights[name][0].cpu(), torch.randn(1, k, generator=gen).to(torch.bfloat16)) for name, n, k in D.shapes()]
    nbytes = D.chain_bytes("bf16")
    sec, passes = _time_passes(lambda: [F.linear(x, w) for w, x in host], budget_s)
    del host
    return {"value": nbytes / sec / 1e9, "unit": "GB/s", "cores": cores, "kind": "reference",
            "sample": (f"torch.nn.functional.linear, bf16, M=1, over the full 113-linear decode-step set "
                       f"({passes} passes, median {sec * 1e3:.1f} ms per set) on {_cpu_name()}"),
            "ms_per_set": sec * 1e3}


def cpu_fp32_set(weights, budget_s: float = 12.0) -> dict:
    """torch F.linear in fp32 on the host cores over the full 113-linear decode-step set (fp32 copies of the bf16
    weights, 5.1 GB), the reference's CPU path at full precision. Bounded: at most 5 passes."""
    import torch
    import torch.nn.functional as F

    from byteprof_amd import decode_set as D

    cores = _cores()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(1)
    host = [(weights[name][0].cpu().float(), torch.randn(1, k, generator=gen)) for name, n, k in D.shapes()]
    sec, passes = _time_passes(lambda: [F.linear(x, w) for w, x in host], budget_s)
    del host
    return {"ms_per_set": sec * 1e3, "cores": cores, "linears": len(D.shapes()),
            "sample": f"the full set, {passes} passes, median"}


def cpu_int8_set(weights8, budget_s: float = 12.0) -> dict:
    """The reference's int8 CPU path over the full 113-linear set: per linear the weights dequantized in the
    activation dtype, then F.linear (byteprof/quant/integrate.py:35-45), on the host cores; at most 5 passes."""
    import torch
    import torch.nn.functional as F

    from byteprof_amd import decode_set as D

    cores = _cores()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(2)
    host = [(weights8[name][0].cpu(), weights8[name][1].cpu(), torch.randn(1, k, generator=gen).to(torch.bfloat16))
            for name, n, k in D.shapes()]

    def one_pass():
        for q, sc, x in host:
            F.linear(x, q.to(x.dtype) * sc.to(x.dtype)[:, None])

    sec, passes = _time_passes(one_pass, budget_s)
    del host
    return {"ms_per_set": sec * 1e3, "cores": cores, "linears": len(D.shapes()),
            "sample": f"the full set, {passes} passes, median; fp16 scales, bf16 activations"}


def mlstm_torch_fp32(c, n, m, q, k, v, i, f, eps: float):
    """The fused multistep recurrence of byteprof/optim/mlstm_multistep.py:21-86 as a torch fp32 step loop over the
    heads at once (DTYPE = DTYPE_STATE = fp32): per step the gates (f_log = log(sigmoid(f)), m_new = max(f_log + m,
    i), f_act, i_act, max_val), C <- f_act C + i_act k v^T, n <- f_act n + i_act k, h = (q_s C) / (max(|q_s . n|,
    max_val) + eps) with q_s = q DQ^-1/2. c [NH, DQ, DV], n [NH, DQ], m [NH]; q, k [T, NH, DQ]; v [T, NH, DV];
    i, f [T, NH]. Returns h [T, NH, DV]."""
    import torch

    t_steps, _, dq = q.shape
    scale = dq ** -0.5
    h = torch.empty(t_steps, v.shape[1], v.shape[2])
    for t in range(t_steps):
        f_log = torch.log(torch.sigmoid(f[t]))
        m_new = torch.maximum(f_log + m, i[t])
        max_val = torch.exp(-m_new)
        f_act = torch.exp(f_log + m - m_new)
        i_act = torch.exp(i[t] - m_new)
        c = f_act[:, None, None] * c + i_act[:, None, None] * (k[t][:, :, None] * v[t][:, None, :])
        n = f_act[:, None] * n + i_act[:, None] * k[t]
        qs = q[t] * scale
        h_num = torch.bmm(qs[:, None, :], c)[:, 0, :]
        qn = (qs * n).sum(-1)
        h[t] = h_num / (torch.maximum(qn.abs(), max_val) + eps)[:, None]
        m = m_new
    return h


def cpu_legs(weights8, fp32_set: dict | None = None, budget_s: float = 12.0) -> dict:
    """Further CPU figures on the host cores: fp32 F.linear over the full set (measured by cpu_fp32_set while the
    bf16 weights exist), the int8 dequantize-then-F.linear set, the 8192 x 2048 linear alone (bf16), and the mLSTM
    block as a torch fp32 step loop (T = 16, NH = 4, DQ = DV = 256)."""
    import torch
    import torch.nn.functional as F

    cores = _cores()
    torch.set_num_threads(cores)
    out = {"cores": cores, "cpu": _cpu_name()}
    if fp32_set is not None:
        out["fp32_set"] = fp32_set
    out["int8_dequant_set"] = cpu_int8_set(weights8, budget_s)
    gen = torch.Generator().manual_seed(1)
    w1 = (torch.randn(8192, 2048, generator=gen) * 0.02).to(torch.bfloat16)
    x1 = torch.randn(1, 2048, generator=gen).to(torch.bfloat16)
    sec1, _ = _time_passes(lambda: [F.linear(x1, w1) for _ in range(10)], 3.0)
    out["c1_bf16_us"] = sec1 / 10 * 1e6
    t, nh, dq, dv = 16, 4, 256, 256
    r = lambda *sh: torch.randn(*sh, generator=gen)  # noqa: E731
    args = (r(nh, dq, dv) * 0.1, r(nh, dq) * 0.1, r(nh), r(t, nh, dq), r(t, nh, dq), r(t, nh, dv), r(t, nh),
            r(t, nh) + 3.0)
    secm, passes = _time_passes(lambda: mlstm_torch_fp32(*args, eps=1e-6), 3.0, max_passes=20)
    out["mlstm_block_us"] = {"value": secm * 1e6, "kind": "reference", "threads": cores,
                             "sample": f"torch fp32 step loop of the multistep recurrence, one 16-step block, "
                                       f"{passes} passes, median"}
    return out


def extra(result: dict, key: str, fn, *args) -> None:
    """Runs one secondary figure; a failure is recorded under its key (the headline line is still printed)."""
    import torch

    log(f"[bench] {key}")
    t0 = time.perf_counter()
    try:
        result[key] = fn(*args)
    except Exception as e:  # noqa: BLE001 - recorded in the output, not hidden
        result[key] = {"error": f"{type(e).__name__}: {e}"}
        log(f"[bench] {key} failed: {e}")
    torch.cuda.empty_cache()
    log(f"[bench] {key} done in {time.perf_counter() - t0:.1f} s")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU figures")
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
    stages = D.build_stages(weights, 1, device, seed=0)
    nbytes = D.chain_bytes("bf16")
    g = graph_of(stages)
    log(f"[bench] 65-launch stage graph: warm-up {WARM_S} s + {a.warmup} replays, timing {a.steps} replays")
    ev_ms, wall_ms = time_runs(g.replay, a.steps, a.warmup)
    del g
    ms = max(ev_ms, wall_ms)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] {ms * 1e3:.1f} us per set, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    log("[bench] per-shape launch times (roofline) and the device-copy ceiling")
    shapes = per_shape(stages, "bf16", 1)
    ceiling = copy_ceiling(device)
    empty_us = D.dispatch_gap_us()
    ops = D.build("bf16", 1, device, seed=0, weights=weights)
    result = {
        "metric": METRIC, "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0, 0.02^2) bf16 weights, unit-RMS N(0,1) activations)",
        "config": {"workload": ("OLMo-2-1B-shaped decode-step linear set at M=1, bf16: 16 x (q,k,v,o 2048->2048; "
                                "gate,up 2048->8192; down 8192->2048) + LM head 2048->100352 (113 linears), as 65 "
                                "stream-ordered skinny launches in one HIP graph (q|k|v and gate|up one launch each)"),
                   "M": 1, "linears": len(D.shapes()), "launches": len(stages), "bytes_per_step": nbytes,
                   "us_per_set": ms * 1e3,
                   "pct_of_hbm_peak": gbs / HBM_PEAK_GBS * 100, "event_ms": ev_ms, "wall_ms": wall_ms,
                   "empty_launch_us": empty_us},
        "copy_ceiling": ceiling,
        "roofline": roofline_of_graph(shapes),
        "kernels": shapes,
    }
    del stages
    if not a.no_extras:
        def graph_113():
            g113 = graph_of(ops)
            e113, _ = time_runs(g113.replay, 50)
            del g113
            return {**figures(e113, nbytes), "launches": len(ops), "kernels": per_shape(ops, "bf16", 1)}

        extra(result, "graph_113", graph_113)
        extra(result, "one_launch_set", one_launch, "bf16", weights, nbytes, device, 4, "one-launch-bf16")
        extra(result, "dependent", dependent_figures, "bf16", weights, nbytes, device)
        one = result.get("one_launch_set", {})
        if "gbs" in one:
            # what stream-ordered launches allow: every launch's empty-launch cost plus the set's bytes at the best
            # read rate measured here (the one-launch grid over the same weights)
            result["config"]["floor_us_stream_ordered"] = len(D.stage_shapes()) * empty_us + nbytes / one["gbs"] / 1e3
    del ops
    fp32_set = None
    if not a.no_cpu:
        log("[bench] CPU baseline")
        result["cpu_baseline"] = cpu_baseline(weights)
        if not a.no_extras:
            log("[bench] CPU fp32 set")
            fp32_set = cpu_fp32_set(weights)
    del weights
    torch.cuda.empty_cache()
    if not a.no_extras:
        w8 = D.make_weights("int8", device, seed=0)
        nb8 = D.chain_bytes("int8")

        def int8_set():
            st8 = D.build_stages(w8, 1, device, seed=0)
            gs8 = graph_of(st8)
            es8, _ = time_runs(gs8.replay, 50)
            del gs8
            ops8 = D.build("int8", 1, device, seed=0, weights=w8)
            g8 = graph_of(ops8)
            e8, _ = time_runs(g8.replay, 50)
            del g8
            out = {"bytes_per_step": nb8, "scales": "fp16 per output row",
                   "stage_graph": {**figures(es8, nb8), "launches": len(st8),
                                   "roofline": roofline_of_graph(per_shape(st8, "int8", 1))},
                   "graph_113": {**figures(e8, nb8), "kernels": per_shape(ops8, "int8", 1)},
                   "graph_113_m4": graph_set("int8", w8, 4, device), "graph_113_m16": graph_set("int8", w8, 16, device),
                   "one_launch_set": one_launch("int8", w8, nb8, device, 2, "one-launch-int8"),
                   "dependent": dependent_figures("int8", w8, nb8, device)}
            bf = result
            out["bf16_over_int8_time"] = {
                "stage_graph": bf["config"]["us_per_set"] / out["stage_graph"]["us_per_set"],
                "graph_113": (bf["graph_113"]["us_per_set"] / out["graph_113"]["us_per_set"]
                              if "us_per_set" in bf.get("graph_113", {}) else None),
                "one_launch_set": (bf["one_launch_set"]["us_per_set"] / out["one_launch_set"]["us_per_set"]
                                   if "us_per_set" in bf.get("one_launch_set", {}) else None),
                "dependent_skinny_stage_graph": (bf["dependent"]["skinny_stage_graph"]["us_per_set"]
                                                 / out["dependent"]["skinny_stage_graph"]["us_per_set"]
                                                 if "skinny_stage_graph" in bf.get("dependent", {}) else None)}
            del st8, ops8
            return out

        extra(result, "int8_set", int8_set)
        if not a.no_cpu:
            extra(result, "cpu_legs", cpu_legs, w8, fp32_set)
        del w8
        torch.cuda.empty_cache()
        extra(result, "int4", int4_figures, device)
        extra(result, "c1", c1_figures, device)
        extra(result, "mlstm", mlstm_block, device)
        extra(result, "sweep_bf16", sweep, device, "bf16")
        extra(result, "sweep_int8", sweep, device, "int8")
        extra(result, "decode_loop", decode_loop, device)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
