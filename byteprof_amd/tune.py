"""Tile-configuration tuner of the skinny kernels on the GPU; writes byteprof_amd/optim/skinny_cfg.json.

The measurement follows the reference's method (byteprof tools/skinny_bench.py:45-71, tools/skinny_tune.py:30-93):
a ring of distinct weight sets applied to one activation block inside a HIP graph, so the weights are streamed from
HBM and not served from cache, the median of several trials per configuration. The ring here is sized against
MI355X's 256 MB Infinity Cache (at least 1 GiB of weights per cell) instead of a 3 MB L2.

bf16 / int8 (the matrix-core kernel of every row count): per (kind, N, K) the tuner keeps ONE K order -- (waves,
split) -- for every activation-row bucket, so an output row stays bitwise independent of M. It times every
(waves, split) at one row (the decode metric) and at 16 rows (the verify widths), each with its best weight blocks
per workgroup and xstage flags (activation staging; the straight-line kernel of the segment count or the general
loop), and at one row with a norm prologue (split 1). It keeps the fastest one-row order; like the reference, a
split > 1 must win by more than 3%; when that order has no split, the split-1 order within 5% of it whose plain and
prologue launches are fastest together (the decode step runs the prologue form); then, among the orders within 2%
of that, the fastest at 16 rows. Then, at that K order, it picks the weight blocks per workgroup and
the flags for each bucket (1; 8: four and eight rows together; 16: nine and sixteen rows, the row groups over one
staged copy among its plans; 32, 64; `--plans-only 16` retunes just those buckets in an existing table). Last, for
launches with a norm prologue (bp_skinny_mf_pro: the decode loops' q|k|v, gate|up and LM head launches), the weight
blocks per workgroup at the same K order, for buckets 1 and 8 (rb_pro; `--pro-only` retunes just those).

Usage: python -m byteprof_amd.tune [--shapes N:K,...] [--kinds bf16,int8,int4] [--out path] [--pro-only]
                                   [--plans-only BUCKETS]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from pathlib import Path

import torch

from .optim import skinny as S
from .quant.hip_int8 import quantize_rowwise_int8

RING_BYTES = 1 << 30
DEFAULT_SHAPES = [(2048, 2048), (8192, 2048), (2048, 8192), (100352, 2048), (6144, 2048), (16384, 2048),
                  (100352, 8192), (8192, 8192)]
WAVES = (1, 2, 4, 8)
SPLITS = (1, 2, 4)
RBS = (1, 2, 4)
INT4_WAVES = (1, 2, 4, 8)


def _ring(kind: str, n: int, k: int, device) -> list[tuple]:
    per = n * k * (2 if kind == "bf16" else 1)
    count = max(2, min(64, RING_BYTES // per))
    g = torch.Generator(device=device).manual_seed(n * 31 + k)
    ring = []
    for _ in range(count):
        w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        ring.append((w,) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16))
    return ring


def _time_calls(calls, trials: int = 5) -> float:
    """us per call: one graph holding the calls (one per ring member), median over trials."""
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


def _launcher(kind: str, ring, x, y, rb: int, waves: int, split: int, xs: int):
    """Calls of the kernel with an explicit plan (rb, waves, split, staging) over the ring."""
    from . import _lib

    L = _lib.lib()
    m, k = x.shape
    n = y.shape[1]
    ws = torch.empty(max(1, split * m * n), dtype=torch.float32, device=x.device)

    def call(a):
        sc, sdt = (a[1].data_ptr(), _lib.TORCH_DT[a[1].dtype]) if kind == "int8" else (None, 0)
        rc = L.bp_skinny_mf(S._KIND_CODE[kind], x.data_ptr(), a[0].data_ptr(), sc, sdt, y.data_ptr(), m, n, k, rb,
                            waves, split, xs, ws.data_ptr(), ws.numel() * 4, _lib.stream_ptr(x.device))
        _lib.check(rc, "bp_skinny_mf")

    return [lambda a=a: call(a) for a in ring]


def _plans(kind: str, m: int, k: int, waves: int, split: int):
    """(rb, xstage flags) of every compiled plan at this K order: staged activations or not, and where the
    straight-line kernel of the segment count applies, that kernel or the general loop (XS_GENERAL)."""
    fixed = S.segments_per_wave(kind, k, waves, split) > 0
    rows = (S.XS_STAGE | S.XS_ROWS2, S.XS_STAGE | S.XS_ROWS4) if 8 < m <= 16 else ()
    for rb in RBS:
        for xs in (0, S.XS_STAGE, S.XS_GENERAL, S.XS_STAGE | S.XS_GENERAL, *rows):
            if xs & S.XS_STAGE and (m > 16 or S._stage_bytes(kind, m, k, split, xs) < 0):
                continue
            if xs & S.XS_GENERAL and not fixed:
                continue
            if S._supported(kind, m, rb, waves, xs & (S.XS_STAGE | S.XS_ROWS)):
                yield rb, xs


def _best_plan(kind, ring, x, y, waves, split, rows_list) -> tuple[float, int, int]:
    """(summed us over the row counts, rb, staging) of the best plan at this K order."""
    best = None
    for rb, xs in _plans(kind, max(rows_list), x.shape[1], waves, split):
        t = sum(_time_calls(_launcher(kind, ring, x[:m].contiguous(), y[:m], rb, waves, split, xs))
                for m in rows_list)
        if best is None or t < best[0]:
            best = (t, rb, xs)
    return best


PRO_BUCKETS = {1: (1,), 8: (2, 4)}  # the row buckets (and row counts timed) where the decode loops run norm prologues


def tune_pro(kind: str, n: int, k: int, entry: dict, device, log=print) -> dict:
    """rb_pro: the weight blocks per workgroup of launches with a norm prologue (bp_skinny_mf_pro, BP_PRO_NORM with
    a residual, as the decode step's q|k|v, gate|up and LM head launches run) at the table's K order, per row bucket
    where the rows stage in LDS; {} where the order splits K (no prologue there)."""
    waves, split = int(entry["waves"]), int(entry.get("split", 1))
    if split != 1:
        return {}
    ring = _ring(kind, n, k, device)
    g = torch.Generator(device=device).manual_seed(n + k)
    x = torch.randn(4, k, generator=g, device=device).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(k, generator=g, device=device)).to(torch.bfloat16)
    res = torch.randn(4, k, generator=g, device=device).to(torch.bfloat16)
    xout = torch.empty(4, k, dtype=torch.bfloat16, device=device)
    y = torch.empty(4, n, dtype=torch.bfloat16, device=device)
    out = {}
    for bucket, rows in PRO_BUCKETS.items():
        if S._stage_bytes(kind, max(rows), k, 1) < 0:  # the rows must stage in LDS
            continue
        best = None
        for rb in RBS:
            if not S._supported(kind, max(rows), rb, waves, True):
                continue
            t = 0.0
            for m in rows:
                calls = [lambda a=a, m=m: S.prologue_mm(x[:m], a[0], a[1] if kind == "int8" else None, y[:m],
                                                        S.PRO_NORM, gamma=gamma, residual=res[:m], xout=xout[:m],
                                                        eps=1e-6, cfg=(8 * rb, waves, 1))
                         for a in ring]
                t += _time_calls(calls)
            if best is None or t < best[0]:
                best = (t, rb)
        if best is not None:
            out[str(bucket)] = best[1]
    log(f"  {kind} {n}x{k}: rb_pro={out}")
    del ring
    torch.cuda.empty_cache()
    return out


def _pro_time(kind: str, ring, x, n: int, k: int, waves: int) -> float | None:
    """us of the best norm-prologue launch (BP_PRO_NORM with a residual, M = 1) at (waves, split 1), or None where
    the row does not stage in LDS."""
    if S._stage_bytes(kind, 1, k, 1) < 0:
        return None
    g = torch.Generator(device=x.device).manual_seed(7)
    gamma = (1 + 0.1 * torch.randn(k, generator=g, device=x.device)).to(torch.bfloat16)
    res = torch.randn(1, k, generator=g, device=x.device).to(torch.bfloat16)
    xout = torch.empty(1, k, dtype=torch.bfloat16, device=x.device)
    y = torch.empty(1, n, dtype=torch.bfloat16, device=x.device)
    x1 = x[:1].contiguous()
    best = None
    for rb in RBS:
        if not S._supported(kind, 1, rb, waves, True):
            continue
        t = _time_calls([lambda a=a: S.prologue_mm(x1, a[0], a[1] if kind == "int8" else None, y, S.PRO_NORM,
                                                   gamma=gamma, residual=res, xout=xout, eps=1e-6,
                                                   cfg=(8 * rb, waves, 1)) for a in ring])
        best = t if best is None or t < best else best
    return best


# the row buckets of a plan and the row counts its choice is timed at (16: a drafting verify round's 9 rows too)
BUCKET_ROWS = ((1, [1]), (8, [4, 8]), (16, [9, 16]), (32, [32]), (64, [64]))


def retune_plans(kind: str, n: int, k: int, entry: dict, buckets, device, log=print) -> dict:
    """The plans (rb, xstage flags) of the given row buckets at the entry's K order (its waves and split), with
    their times; the rest of the entry is kept."""
    waves, split = int(entry["waves"]), int(entry.get("split", 1))
    ring = _ring(kind, n, k, device)
    x = torch.randn(64, k, device=device).to(torch.bfloat16)
    y = torch.empty(64, n, dtype=torch.bfloat16, device=device)
    out = {**entry, "rb": dict(entry.get("rb", {})), "xs": dict(entry.get("xs", {})), "us": dict(entry.get("us", {}))}
    for bucket, rows in BUCKET_ROWS:
        if bucket not in buckets:
            continue
        _, rb, xs = _best_plan(kind, ring, x, y, waves, split, rows)
        out["rb"][str(bucket)], out["xs"][str(bucket)] = rb, xs
        for m in rows:
            out["us"][str(m)] = round(_time_calls(_launcher(kind, ring, x[:m].contiguous(), y[:m], rb, waves, split,
                                                            xs)), 3)
        log(f"  {kind} {n}x{k} bucket {bucket}: rb {rb} xs {xs}: " + ", ".join(f"M={m} {out['us'][str(m)]} us"
                                                                           for m in rows))
    del ring
    torch.cuda.empty_cache()
    return out


def tune_shape(kind: str, n: int, k: int, device, log=print) -> dict:
    ring = _ring(kind, n, k, device)
    nseg = -(-k // S.k_segment(kind))
    x = torch.randn(64, k, device=device).to(torch.bfloat16)
    y = torch.empty(64, n, dtype=torch.bfloat16, device=device)
    orders, pro = {}, {}
    for waves in WAVES:
        for split in SPLITS:
            if waves * split > nseg:
                continue
            t1 = _best_plan(kind, ring, x, y, waves, split, [1])
            t16 = _best_plan(kind, ring, x, y, waves, split, [16])
            orders[(waves, split)] = (t1[0], t16[0])
            if split == 1:
                pro[(waves, split)] = _pro_time(kind, ring, x, n, k, waves)
            tp = pro.get((waves, split))
            log(f"  {kind} {n}x{k} waves={waves} split={split}: M=1 {t1[0]:.2f} us (rb {t1[1]}, xs {t1[2]}), "
                f"M=16 {t16[0]:.2f} us (rb {t16[1]}, xs {t16[2]})" + (f", with a norm prologue {tp:.2f} us" if tp else ""))
    best = min(orders, key=lambda o: orders[o][0])
    if best[1] > 1:
        no_split = min((o for o in orders if o[1] == 1), key=lambda o: orders[o][0])
        if orders[no_split][0] <= orders[best][0] * 1.03:
            best = no_split
    if best[1] == 1 and pro.get(best) is not None:
        # among split-1 orders within 5% at one row, the one fastest as a plain launch and with a norm prologue
        # together (the decode step runs the prologue form of its q|k|v, gate|up and head launches)
        cand = [o for o in orders if o[1] == 1 and pro.get(o) is not None and orders[o][0] <= orders[best][0] * 1.05]
        best = min(cand, key=lambda o: orders[o][0] + pro[o])
    near = [o for o in orders if orders[o][0] <= orders[best][0] * 1.02 and (o[1] == 1 or best[1] > 1)
            and (pro.get(best) is None or (pro.get(o) is not None and orders[o][0] + pro[o]
                                            <= (orders[best][0] + pro[best]) * 1.02))]
    best = min(near, key=lambda o: orders[o][1])
    waves, split = best
    rb, xs, us = {}, {}, {}
    for bucket, rows in BUCKET_ROWS:
        t, rb[str(bucket)], xs[str(bucket)] = _best_plan(kind, ring, x, y, waves, split, rows)
        for m in rows:
            us[str(m)] = round(_time_calls(_launcher(kind, ring, x[:m].contiguous(), y[:m], rb[str(bucket)], waves,
                                                     split, xs[str(bucket)])), 3)
    per = n * k * (2 if kind == "bf16" else 1)
    entry = {"waves": waves, "split": split}
    rb_pro = tune_pro(kind, n, k, entry, device, log)
    log(f"  {kind} {n}x{k}: waves={waves} split={split} rb={rb} xs={xs} us={us} "
        f"(M=1: {per / us['1'] / 1e3:.0f} GB/s of weights)")
    del ring
    torch.cuda.empty_cache()
    return {"waves": waves, "split": split, "rb": rb, "xs": xs, "us": us, **({"rb_pro": rb_pro} if rb_pro else {})}


def tune_int4(n: int, k: int, device, log=print, tiles=S.INT4_TILES) -> dict | None:
    """int4: per tile rows (16, 32, 64: a packing choice), (waves, split) by the M = 1 time (split > 1 kept only if
    it wins by more than 3%); the tile rows of the fastest plan are the entry's, with the time of every row bucket
    at that plan's K order."""
    if k % S.GROUP:
        return None
    groups = k // S.GROUP
    per = n * k // 2
    count = max(2, min(64, RING_BYTES // per))
    x16 = torch.randn(16, k, device=device).to(torch.bfloat16)
    y = torch.empty(16, n, dtype=torch.bfloat16, device=device)
    x1, y1 = x16[:1].contiguous(), y[:1]
    plans, best_tile, us = {}, None, {}
    for tr in tiles:
        g = torch.Generator(device=device).manual_seed(n * 17 + k)
        ring = []
        for _ in range(count):
            w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
            ring.append(S.quantize_int4(w, tr))
            del w
        results = {}
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
        plans[str(tr)] = {"waves": best[0], "split": best[1], "us1": round(results[best], 3)}
        log(f"  int4 {n}x{k} tile {tr}: waves={best[0]} split={best[1]}: {results[best]:.3f} us at M=1")
        if best_tile is None or results[best] < plans[str(best_tile)]["us1"]:
            best_tile = tr
            us = {}
            for bm in (1, 2, 4, 8, 16):
                xb, yb = x16[:bm].contiguous(), y[:bm]
                us[str(bm)] = round(_time_calls([lambda a=a: S.skinny_mm(xb, *a, out=yb, cfg=best) for a in ring]), 3)
        del ring
        torch.cuda.empty_cache()
    top = plans[str(best_tile)]
    log(f"  int4 {n}x{k}: tile rows {best_tile}, waves={top['waves']} split={top['split']}: us {us} "
        f"(M=1: {per / us['1'] / 1e3:.0f} GB/s of codes)")
    return {"tile_rows": best_tile, "waves": top["waves"], "split": top["split"], "us": us, "tiles": plans}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default=None, help="N:K,N:K,... (default: the decode-step set shapes)")
    ap.add_argument("--kinds", default="bf16,int8")
    ap.add_argument("--out", default=str(S._CFG_FILE))
    ap.add_argument("--plans-only", default=None,
                    help="comma-separated row buckets: only (re)tune those buckets' plans (rb, xstage) of the table's "
                         "existing bf16 / int8 entries (the K orders kept)")
    ap.add_argument("--pro-only", action="store_true",
                    help="only (re)tune rb_pro of the table's existing bf16 / int8 entries (the K orders kept)")
    a = ap.parse_args(argv)
    shapes = DEFAULT_SHAPES if a.shapes is None else [tuple(int(v) for v in s.split(":")) for s in a.shapes.split(",")]
    device = torch.device("cuda:0")
    out = Path(a.out)
    table = json.loads(out.read_text()) if out.exists() else {}
    table["_about"] = ("skinny kernel configurations for gfx950, tuned by python -m byteprof_amd.tune. kind|N|K "
                       "(bf16, int8): waves and split of the matrix-core kernel (they fix the K order for every row "
                       "count), rb = 8-row weight blocks per workgroup and xs = xstage flags (1: activations "
                       "staged in LDS, 2: the general segment loop instead of the straight-line kernel of the "
                       "segment count), per row bucket (1, 8, 16, 32, 64), rb_pro = rb of launches with a norm "
                       "prologue (buckets 1 and 8), us = measured time per call by row count (ring of distinct "
                       "weights, HIP graph); int4|N|K: tile_rows = the rows per tile to pack the weight "
                       "with, waves and split of the int4 kernel at those tile rows, us per row count, and tiles = the "
                       "best (waves, split) and its M = 1 time for each tile rows.")
    log = lambda m: print(m, flush=True)  # noqa: E731
    if a.plans_only:
        buckets = {int(b) for b in a.plans_only.split(",")}
        for kind in a.kinds.split(","):
            for n, k in shapes:
                key = f"{kind}|{n}|{k}"
                if kind == "int4" or key not in table:
                    continue
                print(f"[tune] {key} plans of buckets {sorted(buckets)}", flush=True)
                table[key] = retune_plans(kind, n, k, table[key], buckets, device, log=log)
                out.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")
        print(f"[tune] wrote {out}")
        return 0
    if a.pro_only:
        for kind in a.kinds.split(","):
            for n, k in shapes:
                key = f"{kind}|{n}|{k}"
                if kind == "int4" or key not in table:
                    continue
                print(f"[tune] {key} rb_pro", flush=True)
                rb_pro = tune_pro(kind, n, k, table[key], device, log=log)
                if rb_pro:
                    table[key]["rb_pro"] = rb_pro
                else:
                    table[key].pop("rb_pro", None)
                out.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")
        print(f"[tune] wrote {out}")
        return 0
    for kind in a.kinds.split(","):
        for n, k in shapes:
            print(f"[tune] {kind} {n}x{k}", flush=True)
            e = tune_int4(n, k, device, log=log) if kind == "int4" else tune_shape(kind, n, k, device, log=log)
            if e is not None:
                table[f"{kind}|{n}|{k}"] = e
                out.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")  # after every cell (resumable)
    print(f"[tune] wrote {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
