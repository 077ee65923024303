"""Short GPU programs to run under rocprofv3 (kernel trace, HBM counters).

  python -m byteprof_amd.profiling set  [--kind bf16|int8] [--replays R]   the decode-step set as its 65 stage
                                                                         launches in one graph, R replays
  python -m byteprof_amd.profiling set113 [--kind bf16|int8] [--replays R] the same as 113 launches (one per linear)
  python -m byteprof_amd.profiling chain [--kind bf16|int8] [--dependent] [--waves W] [--replays R]
                                                                         the set as one launch (independent linears,
                                                                         or the dependent stages), R launches
  python -m byteprof_amd.profiling stages [--kind bf16|int8] [--replays R]
                                                                         the dependent set as 65 stream-ordered
                                                                         launches (one per stage), R passes
  python -m byteprof_amd.profiling decode [--kind bf16|int8] [--tokens N] [--draft]
                                                                         the graph-captured greedy decode loop
                                                                         of the OLMo-2-1B shape, 8 prompt + N tokens;
                                                                         --draft: then the drafting loop with the
                                                                         oracle drafter (K up to 8)
  python -m byteprof_amd.profiling skinny [--kind bf16|int8|int4] [--n N] [--k K] [--m M] [--replays R]
                                                                         skinny_mm over a ring of distinct weights
  python -m byteprof_amd.profiling mlstm [--replays R]                    the fused mLSTM multistep (4 heads,
                                                                         256 x 256, 16 steps), R launches
  python -m byteprof_amd.profiling mlstm-timeline [--replays R]           the same from the timeline library
                                                                         (build --timeline): per-stage times of
                                                                         the workgroups of one launch, R times
  python -m byteprof_amd.profiling skinny-timeline [--kind bf16|int8] [--n N] [--k K] [--m M] [--replays R]
                                                                         skinny_mm (tuned plan) from the timeline
                                                                         library: per-stage times of the matrix-core
                                                                         kernel's workgroups, R launches
  python -m byteprof_amd.profiling copy [--mib 256] [--reps 5]             a device-to-device copy of known size
  python -m byteprof_amd.profiling summarize TRACE_DB [--fetch DB --write DB --fetch-copy DB --write-copy DB
                                             --copy-mib 256]               text summary of rocprofv3 databases

The copy is the calibration reference for the FETCH_SIZE / WRITE_SIZE counters: it reads and writes exactly
`mib` MiB per dispatch, so expected / counter is the factor that turns a counter reading into HBM bytes.
`summarize` needs no GPU: it reads the SQLite databases rocprofv3 writes (kernels / counters_collection views).
"""

from __future__ import annotations

import argparse
import os
import sys

import torch


def _kernel_stats(db_path: str) -> list[tuple[str, int, int, float, float, float]]:
    """(kernel name, grid threads, calls, total us, average us, median us) from a kernel-trace database, longest
    total first; the grid size tells the launches of one kernel instantiation on different shapes apart."""
    import sqlite3
    import statistics

    cur = sqlite3.connect(db_path).cursor()
    groups: dict[tuple[str, int], list[float]] = {}
    for name, grid, dur in cur.execute("select name, grid_x * grid_y * grid_z, duration from kernels"):
        groups.setdefault((name, int(grid)), []).append(dur / 1e3)
    out = [(n, gs, len(d), sum(d), sum(d) / len(d), statistics.median(d)) for (n, gs), d in groups.items()]
    return sorted(out, key=lambda r: -r[3])


def _counter_avgs(db_path: str) -> dict[tuple[str, int], tuple[str, int, float]]:
    """(kernel name, grid size) -> (counter, dispatches, average value in KiB per dispatch). The grid size tells the
    launches of one kernel instantiation on different shapes apart."""
    import sqlite3

    cur = sqlite3.connect(db_path).cursor()
    rows = cur.execute("select kernel_name, grid_size, counter_name, count(*), avg(value) from counters_collection "
                       "group by kernel_name, grid_size, counter_name").fetchall()
    return {(n, int(gs)): (c, int(k), v) for n, gs, c, k, v in rows}


def _counter_table(db_path: str) -> dict[tuple[str, int], dict[str, tuple[int, float]]]:
    """(kernel name, grid size) -> {counter: (dispatches, average value per dispatch)} for every counter of a
    --pmc database (derived metrics such as MfmaUtil included)."""
    import sqlite3

    cur = sqlite3.connect(db_path).cursor()
    rows = cur.execute("select kernel_name, grid_size, counter_name, count(*), avg(value) from counters_collection "
                       "group by kernel_name, grid_size, counter_name").fetchall()
    out: dict[tuple[str, int], dict[str, tuple[int, float]]] = {}
    for n, gs, c, k, v in rows:
        out.setdefault((n, int(gs)), {})[c] = (int(k), float(v))
    return out


def _short(name: str) -> str:
    return name.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")


def summarize(a) -> int:
    print("## kernel trace (rocprofv3 --kernel-trace --stats)")
    print(f"{'kernel':<72} {'grid threads':>12} {'calls':>7} {'total us':>11} {'avg us':>9} {'median us':>10}")
    for name, grid, calls, tot, avg, med in _kernel_stats(a.db):
        if a.all or "bp::" in name:
            print(f"{_short(name)[:72]:<72} {grid:>12} {calls:>7} {tot:>11.1f} {avg:>9.3f} {med:>10.3f}")
    for db in a.pmc or []:
        print()
        print(f"## counters per dispatch ({db.split('/')[-2] if '/' in db else db})")
        for (name, grid), counters in sorted(_counter_table(db).items()):
            if "bp::" not in name and not a.all:
                continue
            vals = ", ".join(f"{c} {v:.4g}" for c, (_, v) in sorted(counters.items()))
            print(f"{_short(name)[:64]:<64} grid {grid:>9}: {vals}")
    if not a.fetch:
        return 0
    expected_kib = a.copy_mib * 1024
    fetch_copy = [v for (n, _), v in _counter_avgs(a.fetch_copy).items() if "copy" in n.lower()][0][2]
    write_copy = [v for (n, _), v in _counter_avgs(a.write_copy).items() if "copy" in n.lower()][0][2]
    f_scale, w_scale = expected_kib / fetch_copy, expected_kib / write_copy
    print()
    print(f"## HBM counters (KiB per dispatch), calibrated on a {a.copy_mib} MiB device copy")
    print(f"copy: FETCH_SIZE {fetch_copy:.1f} KiB -> scale {f_scale:.4f}; WRITE_SIZE {write_copy:.1f} KiB "
          f"-> scale {w_scale:.4f}")
    fetch, write = _counter_avgs(a.fetch), _counter_avgs(a.write)
    print(f"{'kernel':<72} {'grid threads':>12} {'dispatches':>10} {'FETCH KiB':>11} {'WRITE KiB':>10} "
          f"{'traffic MB':>11}")
    for key in sorted(fetch):
        name, grid = key
        if "bp::" not in name and not a.all:
            continue
        _, k, fv = fetch[key]
        wv = write.get(key, ("", 0, 0.0))[2]
        traffic = (fv * f_scale + wv * w_scale) * 1024 / 1e6
        print(f"{_short(name)[:72]:<72} {grid:>12} {k:>10} {fv:>11.1f} {wv:>10.1f} {traffic:>11.3f}")
    if a.chain_tag:
        kernel = "chain_kernel"
        print()
        print(f"## traffic per launch of the {kernel}, {a.chain_tag} (bytes; read by bench.py)")
        for key in sorted(fetch):
            if kernel in key[0]:
                nbytes = (fetch[key][2] * f_scale + write.get(key, ("", 0, 0.0))[2] * w_scale) * 1024
                print(f"traffic: {_short(key[0]).replace('bp::', '')} {a.chain_tag} {nbytes:.0f}")
    if a.set_kind:
        print()
        print(f"## traffic per launch of the {a.set_kind} decode-step set shapes (bytes; read by bench.py)")
        for (kernel, shape), grid in _set_launches(a.set_kind).items():
            for key in fetch:
                if key[1] == grid and _short(key[0]).replace("bp::", "") == kernel:
                    nbytes = (fetch[key][2] * f_scale + write.get(key, ("", 0, 0.0))[2] * w_scale) * 1024
                    print(f"traffic: {kernel} {shape} {nbytes:.0f}")
    return 0


def _set_launches(kind: str) -> dict[tuple[str, str], int]:
    """(kernel instantiation, 'NxK') -> grid threads of the decode-step set's launches at M = 1 (the 65 stage
    launches and the 113 per-linear launches)."""
    from . import decode_set as D
    from .optim import skinny as S

    out = {}
    for _, n, k in D.shapes() + D.stage_shapes():
        rb, waves, split, _ = S._resolve(kind, n, k, 1, None)
        grid = -(-n // (8 * rb)) * waves * 64 * split
        out[(D.kernel_key(kind, n, k, 1), f"{n}x{k}")] = grid
    return out


MLSTM_STAGES = ("entry -> first group's loads landed", "gate chain (m_t, activations)", "16 positions' updates",
                "in-wave reductions", "cross-wave combine (LDS, barrier)", "outputs stored (barrier)", "end")


def mlstm_timeline(a, device) -> int:
    """Per-stage times of the fused mLSTM multistep's workgroups from the timeline library's s_memrealtime stamps
    (thread 0 of each workgroup; 100 MHz, 10 ns resolution): medians over the workgroups of one launch of a graph
    of 64 launches, the spread of the workgroups' starts and the launch's span, and the graph's time per launch."""
    import ctypes
    import statistics

    import numpy as np

    from . import _lib
    from . import decode_set as D
    from .optim import draft_fused

    lib = _lib.lib()
    if not hasattr(lib, "bp_mlstm_timeline_read"):
        print(f"{os.environ[_lib.LIB_ENV]} has no timeline: build it with python -m byteprof_amd.build --timeline",
              file=sys.stderr)
        return 1
    read = lib.bp_mlstm_timeline_read
    read.restype, read.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t]
    g = torch.Generator(device=device).manual_seed(0)
    t, nh, dq, dv = 16, 4, 256, 256
    r = lambda *shape: torch.randn(*shape, generator=g, device=device)  # noqa: E731
    q, k, v = (r(t, nh, d).to(torch.bfloat16) for d in (dq, dq, dv))
    i, f = r(t, nh, 1), r(t, nh, 1) + 3.0
    state = (r(1, nh, dq, dv) * 0.1, r(1, nh, dq) * 0.1, r(1, nh, 1))
    h = torch.empty(t, nh, dv, dtype=torch.bfloat16, device=device)
    ns, ms = torch.empty(nh, dq, device=device), torch.empty(nh, device=device)
    gr = D.capture([lambda: draft_fused.multistep_fw(state, q, k, v, i, f, h, ns, ms, eps=1e-6)] * 64)
    D.time_replays(gr, 3, 1)
    us = statistics.median(D.time_replays(gr, 10, 5)) * 1000 / 64
    print(f"mLSTM multistep (NH {nh}, {dq} x {dv}, T {t}, bf16), timeline library: {us:.3f} us per launch in a graph "
          f"of 64 launches")
    buf = np.zeros((1024, 8), np.uint64)
    wgs = nh * dv // draft_fused.BV
    for rep in range(a.replays):
        gr.replay()
        torch.cuda.synchronize()
        _lib.check(read(buf.ctypes.data, buf.nbytes), "bp_mlstm_timeline_read")
        ts = (buf[:wgs].astype(np.int64) - int(buf[:wgs, 0].min())) * 10  # ns from the first workgroup's start
        med = [float(np.median(ts[:, e + 1] - ts[:, e])) for e in range(7)]
        print(f"launch {rep}: {wgs} workgroups, starts spread over {ts[:, 0].max()} ns, span {ts[:, 7].max()} ns; "
              "per-workgroup medians (ns): " + "; ".join(f"{n} {m:.0f}" for n, m in zip(MLSTM_STAGES, med)))
    return 0


MF_STAGES = ("entry -> first loads issued", "-> first segment's MFMAs", "-> last segment's MFMAs",
             "-> tiles in LDS (barrier)", "-> outputs issued", "-> stores done")


def skinny_timeline(a, device) -> int:
    """Per-stage times of the matrix-core skinny kernel's workgroups (the timeline library's s_memrealtime stamps,
    thread 0 of each workgroup, 100 MHz): skinny_mm with the tuned plan over a ring of distinct weights (streamed
    from HBM) in one HIP graph, replayed R times; after each replay, the last launch's workgroups: the spread of
    their starts, the launch's span and the per-workgroup medians of each stage."""
    import ctypes

    import numpy as np

    from . import _lib
    from .optim import skinny as S
    from .quant.hip_int8 import quantize_rowwise_int8

    lib = _lib.lib()
    if not hasattr(lib, "bp_mf_timeline_read"):
        print(f"{os.environ.get(_lib.LIB_ENV)} has no timeline: build it with python -m byteprof_amd.build "
              "--timeline", file=sys.stderr)
        return 1
    read = lib.bp_mf_timeline_read
    read.restype, read.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t]
    per = a.n * a.k * (2 if a.kind == "bf16" else 1)
    ring = []
    for _ in range(max(2, int((a.ring_mib << 20) // per))):
        w = (torch.randn(a.n, a.k, device=device) * 0.02).to(torch.bfloat16)
        ring.append((w,) if a.kind == "bf16" else quantize_rowwise_int8(w, torch.float16))
        del w
    x = torch.randn(a.m, a.k, device=device).to(torch.bfloat16)
    y = torch.empty(a.m, a.n, dtype=torch.bfloat16, device=device)
    rb, waves, split, xs = S._resolve(a.kind, a.n, a.k, a.m, None)
    wgs = -(-a.n // (8 * rb)) * split
    from . import decode_set as D

    g = D.capture([lambda args=args: S.skinny_mm(x, *args, out=y) for args in ring])
    D.time_replays(g, 2, 1)
    us = float(np.median(D.time_replays(g, 5, 3))) * 1000 / len(ring)
    print(f"skinny_mm {a.kind} {a.n}x{a.k} at M={a.m}: plan rb {rb} waves {waves} split {split} xstage {xs}, "
          f"{wgs} workgroups; a graph of the ring of {len(ring)} weights: {us:.2f} us per launch (timeline build)")
    buf = np.zeros((16384, 8), np.uint64)
    n = min(wgs, buf.shape[0])
    for r in range(a.replays):
        g.replay()  # the stamps are the ring's last launch's, right after the launch before it
        torch.cuda.synchronize()
        _lib.check(read(buf.ctypes.data, buf.nbytes), "bp_mf_timeline_read")
        ts = (buf[:n].astype(np.int64) - int(buf[:n, 0].min())) * 10  # ns from the first workgroup's entry
        med = [float(np.median(ts[:, e + 1] - ts[:, e])) for e in range(6)]
        print(f"launch {r}: starts spread over {ts[:, 0].max()} ns, span {ts[:, 6].max()} ns, workgroup median "
              f"{np.median(ts[:, 6] - ts[:, 0]):.0f} ns; stage medians (ns): "
              + "; ".join(f"{s} {m:.0f}" for s, m in zip(MF_STAGES, med)))
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=("set", "set113", "chain", "stages", "decode", "skinny", "mlstm",
                                     "mlstm-timeline", "skinny-timeline", "copy",
                                     "summarize"))
    ap.add_argument("db", nargs="?", help="summarize: kernel-trace database")
    ap.add_argument("--fetch", help="summarize: FETCH_SIZE database of the workload")
    ap.add_argument("--write", help="summarize: WRITE_SIZE database of the workload")
    ap.add_argument("--fetch-copy", help="summarize: FETCH_SIZE database of the calibration copy")
    ap.add_argument("--write-copy", help="summarize: WRITE_SIZE database of the calibration copy")
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--pmc", action="append", help="summarize: any --pmc database, counters per dispatch")
    ap.add_argument("--all", action="store_true", help="summarize: include kernels outside this library")
    ap.add_argument("--set-kind", choices=("bf16", "int8"), help="summarize: emit traffic lines for the set shapes")
    ap.add_argument("--chain-tag", help="summarize: emit traffic lines for the one-launch set kernel under this tag")
    ap.add_argument("--kind", default="bf16", choices=("bf16", "int8", "int4"))
    ap.add_argument("--dependent", action="store_true", help="chain: stages read the outputs they depend on")
    ap.add_argument("--waves", type=int, default=0, help="chain: waves per workgroup (0: the set's default)")
    ap.add_argument("--replays", type=int, default=5)
    ap.add_argument("--n", type=int, default=100352, help="skinny: output rows")
    ap.add_argument("--k", type=int, default=2048, help="skinny: input length")
    ap.add_argument("--m", type=int, default=16, help="skinny: activation rows")
    ap.add_argument("--ring-mib", type=int, default=1024, help="skinny: MiB of distinct weights in the ring")
    ap.add_argument("--tokens", type=int, default=128, help="decode: new tokens")
    ap.add_argument("--draft", action="store_true", help="decode: also the drafting loop (oracle drafter)")
    ap.add_argument("--mib", type=int, default=256)
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args(argv)
    if a.what == "summarize":
        return summarize(a)
    device = torch.device("cuda:0")
    if a.what == "copy":
        src = torch.empty(a.mib << 20, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        for _ in range(a.reps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copied {a.mib} MiB x {a.reps}", flush=True)
        return 0
    from . import _lib
    from . import decode_set as D

    if a.what in ("mlstm-timeline", "skinny-timeline") and not os.environ.get(_lib.LIB_ENV):
        from . import build as B

        os.environ[_lib.LIB_ENV] = str(B.TIMELINE_LIB_PATH)  # before the first load
    _lib.lib()
    if a.what == "skinny":
        from .optim import skinny as S
        from .quant.hip_int8 import quantize_rowwise_int8

        per = a.n * a.k * {"bf16": 2, "int8": 1, "int4": 0.5}[a.kind]
        ring = []
        # distinct weights past the caches (256 MiB of MALL): streamed from HBM every call
        for r in range(max(2, int((a.ring_mib << 20) // per))):
            w = (torch.randn(a.n, a.k, device=device) * 0.02).to(torch.bfloat16)
            if a.kind == "bf16":
                ring.append((w,))
            elif a.kind == "int8":
                ring.append(quantize_rowwise_int8(w, torch.float16))
            else:
                ring.append(S.quantize_int4(w, S.int4_tile_rows(a.n, a.k)))
            del w
        x = torch.randn(a.m, a.k, device=device).to(torch.bfloat16)
        y = torch.empty(a.m, a.n, dtype=torch.bfloat16, device=device)
        cfg = None
        for _ in range(a.replays):
            for args in ring:
                S.skinny_mm(x, *args, out=y, cfg=cfg)
        torch.cuda.synchronize()
        print(f"skinny_mm {a.kind} {a.n}x{a.k} at M={a.m} (tuned plan): {a.replays} passes "
              f"over {len(ring)} weights", flush=True)
        return 0
    if a.what == "mlstm-timeline":
        return mlstm_timeline(a, device)
    if a.what == "skinny-timeline":
        return skinny_timeline(a, device)
    if a.what == "mlstm":
        from .optim import draft_fused

        g = torch.Generator(device=device).manual_seed(0)
        t, nh, dq, dv = 16, 4, 256, 256
        r = lambda *shape: torch.randn(*shape, generator=g, device=device)  # noqa: E731
        q, k, v = (r(t, nh, d).to(torch.bfloat16) for d in (dq, dq, dv))
        i, f = r(t, nh, 1), r(t, nh, 1) + 3.0
        state = (r(1, nh, dq, dv) * 0.1, r(1, nh, dq) * 0.1, r(1, nh, 1))
        h = torch.empty(t, nh, dv, dtype=torch.bfloat16, device=device)
        ns, ms = torch.empty(nh, dq, device=device), torch.empty(nh, device=device)
        for _ in range(a.replays):
            draft_fused.multistep_fw(state, q, k, v, i, f, h, ns, ms, eps=1e-6)
        torch.cuda.synchronize()
        print(f"mLSTM multistep (NH {nh}, {dq} x {dv}, T {t}): {a.replays} launches", flush=True)
        return 0
    if a.what == "chain":
        ch = D.build_chain(a.kind, device, dependent=a.dependent, waves=a.waves or D.CHAIN_WAVES)
        for _ in range(a.replays):
            ch.lset.run()
        torch.cuda.synchronize()
        if ch.lset.timed_out():
            print("a launch gave up waiting for another workgroup", file=sys.stderr)
            return 1
        print(f"ran the {a.kind} decode-step set as one launch {a.replays} times "
              f"({len(ch.stages)} stages, {'dependent' if a.dependent else 'independent'})", flush=True)
        return 0
    if a.what == "stages":
        ch = D.build_chain(a.kind, device, dependent=True)
        g = D.capture([lc.run for lc in D.stage_launches(ch)])
        for _ in range(a.replays):
            g.replay()
        torch.cuda.synchronize()
        print(f"replayed the {a.kind} dependent set as {len(ch.stages)} stage launches {a.replays} times", flush=True)
        return 0
    if a.what == "decode":
        from .optim import olmo as OG

        dec = OG.OlmoDecoder(OG.OLMO2_1B, OG.random_weights(OG.OLMO2_1B, device, seed=4), a.kind)
        generate = OG.make_generate_graph(dec)
        prompt = torch.tensor([[11, 2027, 5, 99999, 42, 3, 3, 1000]])
        out = generate(prompt, max_new_tokens=a.tokens)
        torch.cuda.synchronize()
        print(f"decoded {out.shape[1] - prompt.shape[1]} tokens ({a.kind}, graph loop)", flush=True)
        if a.draft:
            from .optim import olmo_draft as OD

            key = tuple(prompt[0].tolist())
            truth = {key: out[0, prompt.shape[1]:].tolist()}
            stats = OD.Stats()
            gen, _ = OD.make_generate_draft(dec, {"kind": "oracle", "truth": truth}, stats)
            for _ in range(2):  # the second pass drafts the first pass's own continuation
                res = gen(prompt, max_new_tokens=a.tokens)
                truth[key] = res[0, prompt.shape[1]:].tolist()
            torch.cuda.synchronize()
            print(f"drafting loop: {stats.dump()}", flush=True)
        return 0
    weights = D.make_weights(a.kind, device)
    ops = D.build_stages(weights, 1, device) if a.what == "set" else D.build(a.kind, 1, device, weights=weights)
    g = D.capture(ops)
    for _ in range(a.replays):
        g.replay()
    torch.cuda.synchronize()
    print(f"replayed the {a.kind} decode-step set {a.replays} times ({len(ops)} launches each)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
