"""Tile-configuration tuner of the skinny kernels on the GPU; writes byteprof_amd/optim/skinny_cfg.json.

The measurement follows the reference's method (byteprof tools/skinny_bench.py:45-71, tools/skinny_tune.py:30-93):
a ring of distinct weight sets applied to one activation block inside a HIP graph, so the weights are streamed from
HBM and not served from cache, the median of several trials per configuration. The ring here is sized against
MI355X's 256 MB Infinity Cache (at least 1 GiB of weights per cell) instead of a 3 MB L2.

Per (kind, N, K) the tuner keeps ONE K order (waves, split) for every activation-row bucket of the VALU kernels, so
an output row stays bitwise independent of M: it picks (waves, split) by the M = 1 time (the decode metric), then
the rows per workgroup separately for each bucket. Like the reference, a split > 1 is kept only if it wins by more
than 3%. The matrix-core kernels get one configuration per shape for the 8- and 16-row buckets together ('mfma',
chosen at M = 16, used when it beats the VALU kernels over both buckets).

Usage: python -m byteprof_amd.tune [--shapes N:K,...] [--kinds bf16,int8,int4] [--out path] [--quick] [--mfma-only]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from pathlib import Path

import torch

from . import _lib
from .optim import skinny as S
from .quant.hip_int8 import quantize_rowwise_int8

RING_BYTES = 1 << 30
DEFAULT_SHAPES = [(2048, 2048), (8192, 2048), (2048, 8192), (100352, 2048), (6144, 2048), (16384, 2048),
                  (100352, 8192), (8192, 8192)]
ROWS = (2, 4, 8, 16, 32)
WAVES = (1, 2, 4, 8, 16)
SPLITS = (1, 2, 4)


def _ring(kind: str, n: int, k: int, device) -> list[tuple]:
    per = n * k * (2 if kind == "bf16" else 1)
    count = max(2, min(64, RING_BYTES // per))
    g = torch.Generator(device=device).manual_seed(n * 31 + k)
    ring = []
    for _ in range(count):
        w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        ring.append((w,) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16))
    return ring


def _time_cfg(ring, x, y, cfg, trials: int = 5) -> float:
    """us per call: one graph holding one call per ring member."""
    calls = [lambda a=a: S.skinny_mm(x, *a, out=y, cfg=cfg) for a in ring]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls[:2]:
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(trials):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) * 1000.0 / len(calls))
    del g
    return statistics.median(out)


def _supported(kind: str, bm: int, rows: int, waves: int) -> bool:
    return bool(_lib.lib().bp_skinny_config_supported(S._KIND_CODE[kind], bm, rows, waves))


def tune_shape(kind: str, n: int, k: int, device, quick: bool = False, log=print) -> dict:
    ring = _ring(kind, n, k, device)
    x16 = torch.randn(16, k, device=device).to(torch.bfloat16)
    nch = -(-k // S._CHUNK[kind])
    # 1. K order (waves, split) and rows at M = 1
    x1 = x16[:1].contiguous()
    y1 = torch.empty(1, n, dtype=torch.bfloat16, device=device)
    best = None
    results = {}
    for waves in WAVES:
        if waves > nch:
            continue
        for split in SPLITS:
            if split > 1 and (split > nch // waves or quick):
                continue
            for rows in ROWS:
                if not _supported(kind, 1, rows, waves):
                    continue
                us = _time_cfg(ring, x1, y1, (rows, waves, split))
                results[(rows, waves, split)] = us
                if best is None or us < best[0]:
                    best = (us, rows, waves, split)
    us1, rows1, waves, split = best
    # keep split > 1 only if it wins by more than 3% over the best split-1 configuration
    if split > 1:
        no_split = min((v, r, w) for (r, w, s), v in results.items() if s == 1)
        if no_split[0] <= us1 * 1.03:
            us1, rows1, waves, split = no_split[0], no_split[1], no_split[2], 1
    entry = {"waves": waves, "split": split, "rows": {"1": rows1}, "us": {"1": round(us1, 3)}}
    log(f"  {kind} {n}x{k}: M=1 best rows={rows1} waves={waves} split={split}: {us1:.2f} us "
        f"({(n * k * (2 if kind == 'bf16' else 1)) / us1 / 1e3:.0f} GB/s)")
    # 2. rows for the other buckets at that K order
    for bm in (2, 4, 8, 16):
        xb = x16[:bm].contiguous()
        yb = torch.empty(bm, n, dtype=torch.bfloat16, device=device)
        cands = [(_time_cfg(ring, xb, yb, (r, waves, split)), r) for r in ROWS if _supported(kind, bm, r, waves)]
        us_b, rows_b = min(cands)
        entry["rows"][str(bm)] = rows_b
        entry["us"][str(bm)] = round(us_b, 3)
    log(f"    rows per bucket {entry['rows']} us {entry['us']}")
    del ring
    torch.cuda.empty_cache()
    return entry


MFMA_BLOCK_ROWS = (16, 32, 64)
MFMA_WAVES = (1, 2, 4, 8)
MFMA_DEPTHS = (1, 2)


def _time_calls(calls, trials: int = 5) -> float:
    """us per call: one graph holding the calls."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls[:2]:
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(trials):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) * 1000.0 / len(calls))
    del g
    return statistics.median(out)


def tune_mfma(kind: str, n: int, k: int, device, entry: dict, log=print) -> dict | None:
    """Matrix-core configuration of a shape's 8- and 16-row buckets: (block_rows, waves, depth, split) by the
    16-row time (split > 1 kept only if it wins by more than 3%), then 'use' = whether it beats the VALU kernel
    over both buckets (one family serves both, so rows stay bitwise independent of M within them)."""
    step = S.mfma_k_step(kind)
    if k % step:
        return None
    steps = k // step
    ring = _ring(kind, n, k, device)
    x16 = torch.randn(16, k, device=device).to(torch.bfloat16)
    y16 = torch.empty(16, n, dtype=torch.bfloat16, device=device)
    results = {}
    for br in MFMA_BLOCK_ROWS:
        for w in MFMA_WAVES:
            if w > steps:
                continue
            for d in MFMA_DEPTHS:
                for sp in SPLITS:
                    if sp > 1 and sp * w > steps:
                        continue
                    calls = [lambda a=a: S.launch_mfma(kind, x16, a[0], a[1] if kind == "int8" else None, y16, br, w,
                                                       d, sp) for a in ring]
                    results[(br, w, d, sp)] = _time_calls(calls)
    # the LDS-staged variants: 16-row blocks, the smallest valid split and twice it
    for d in S.STAGED_DEPTHS:
        for w in (1, 2, 4):
            s0 = S.staged_split(kind, k, 1, w, d)
            if s0 is None:
                continue
            for sp in sorted({s0, S.staged_split(kind, k, 2 * s0, w, d)} - {None}):
                calls = [lambda a=a: S.launch_mfma(kind, x16, a[0], a[1] if kind == "int8" else None, y16, 16, w, d,
                                                   sp) for a in ring]
                results[(16, w, d, sp)] = _time_calls(calls)
    best = min(results, key=results.get)
    if best[3] > 1:
        no_split = [c for c in results if c[3] == 1]
        if no_split:
            no_split = min(no_split, key=results.get)
            if results[no_split] <= results[best] * 1.03:
                best = no_split
    br, w, d, sp = best
    us = {"16": round(results[best], 3)}
    x8 = x16[:8].contiguous()
    y8 = y16[:8].contiguous()
    us["8"] = round(_time_calls([lambda a=a: S.launch_mfma(kind, x8, a[0], a[1] if kind == "int8" else None, y8, br,
                                                             w, d, sp) for a in ring]), 3)
    valu = [float(entry["us"][b]) for b in ("8", "16")] if "us" in entry else None
    use = valu is None or us["8"] + us["16"] < valu[0] + valu[1]
    log(f"  {kind} {n}x{k} mfma: block_rows={br} waves={w} depth={d} split={sp}: M=8 {us['8']:.2f} us, "
        f"M=16 {us['16']:.2f} us (VALU {valu}) -> {'mfma' if use else 'valu'}")
    del ring
    torch.cuda.empty_cache()
    return {"block_rows": br, "waves": w, "depth": d, "split": sp, "us": us, "use": use}


INT4_WAVES = (1, 2, 4, 8)


def tune_int4(n: int, k: int, device, log=print) -> dict | None:
    """int4 (tile rows 32, the quantizer's default): (waves, split) by the M = 1 time (split > 1 kept only if it
    wins by more than 3%), then the time of every row bucket at that K order."""
    if k % S.GROUP:
        return None
    groups = k // S.GROUP
    per = n * k // 2
    count = max(2, min(64, RING_BYTES // per))
    g = torch.Generator(device=device).manual_seed(n * 17 + k)
    ring = []
    for _ in range(count):
        w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        ring.append(S.quantize_int4(w))
        del w
    x16 = torch.randn(16, k, device=device).to(torch.bfloat16)
    y = torch.empty(16, n, dtype=torch.bfloat16, device=device)
    results = {}
    x1, y1 = x16[:1].contiguous(), y[:1]
    for w in INT4_WAVES:
        if w > groups:
            continue
        for sp in SPLITS:
            if sp > 1 and sp * w > groups:
                continue
            results[(w, sp)] = _time_calls([lambda a=a: S.skinny_mm(x1, *a, out=y1, cfg=(w, sp)) for a in ring])
    best = min(results, key=results.get)
    if best[1] > 1:
        no_split = min((c for c in results if c[1] == 1), key=results.get)
        if results[no_split] <= results[best] * 1.03:
            best = no_split
    us = {}
    for bm in (1, 2, 4, 8, 16):
        xb, yb = x16[:bm].contiguous(), y[:bm]
        us[str(bm)] = round(_time_calls([lambda a=a: S.skinny_mm(xb, *a, out=yb, cfg=best) for a in ring]), 3)
    log(f"  int4 {n}x{k}: waves={best[0]} split={best[1]}: us {us} (M=1: {per / us['1'] / 1e3:.0f} GB/s of codes)")
    del ring
    torch.cuda.empty_cache()
    return {"waves": best[0], "split": best[1], "us": us}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default=None, help="N:K,N:K,... (default: the decode-step set shapes)")
    ap.add_argument("--kinds", default="bf16,int8")
    ap.add_argument("--out", default=str(S._CFG_FILE))
    ap.add_argument("--quick", action="store_true", help="no split-K candidates")
    ap.add_argument("--mfma-only", action="store_true",
                    help="tune only the matrix-core entries of the 8- and 16-row buckets (keeps the VALU entries)")
    a = ap.parse_args(argv)
    shapes = DEFAULT_SHAPES if a.shapes is None else [tuple(int(v) for v in s.split(":")) for s in a.shapes.split(",")]
    device = torch.device("cuda:0")
    out = Path(a.out)
    table = json.loads(out.read_text()) if out.exists() else {}
    table["_about"] = ("skinny kernel tile configurations for gfx950, tuned by python -m byteprof_amd.tune: key "
                       "kind|N|K; VALU kernels: waves and split fix the K order for every row bucket, rows per "
                       "bucket; 'mfma': the matrix-core configuration (block_rows, waves, depth, split) of the 8- and "
                       "16-row buckets and whether it is used (depth 1, 2: register-fed, steps in flight; 3, 4: "
                       "LDS-staged, each wave owns whole blocks / the waves share each block); int4|N|K: waves and "
                       "split of the int4 kernel (tile rows 32); us = measured time per call (ring of distinct "
                       "weights, HIP graph)")
    for kind in a.kinds.split(","):
        if kind == "int4":
            for n, k in shapes:
                print(f"[tune] int4 {n}x{k}", flush=True)
                e = tune_int4(n, k, device, log=lambda m: print(m, flush=True))
                if e is not None:
                    table[f"int4|{n}|{k}"] = e
                    out.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")
            continue
        for n, k in shapes:
            print(f"[tune] {kind} {n}x{k}", flush=True)
            key = f"{kind}|{n}|{k}"
            log = lambda m: print(m, flush=True)  # noqa: E731
            if not a.mfma_only or key not in table:
                table[key] = tune_shape(kind, n, k, device, a.quick, log=log)
            mf = tune_mfma(kind, n, k, device, table[key], log=log)
            if mf is not None:
                table[key]["mfma"] = mf
            out.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")  # after every cell (resumable)
    print(f"[tune] wrote {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
