"""The OLMo-2-1B-shaped decode-step linear set at M activation rows, as captured HIP graphs of skinny launches.

Per layer (16): q, k, v, o 2048 -> 2048; gate, up 2048 -> 8192; down 8192 -> 2048; then the LM head
2048 -> 100352: 113 linears in decode order, every weight distinct (2.56 GB in bf16, ten times MI355X's 256 MB
Infinity Cache, so nothing is served from cache across replays). Weights ~ N(0, 0.02^2); each linear's input
~ N(0, 1) renormalised to unit RMS. The reference measures the same linears one call each inside a CUDA graph
(byteprof tools/skinny_bench.py:45-71; FINDINGS "OLMo-2 16-block linear set").

The linears of a stage (q|k|v, gate|up) are adjacent rows of one weight allocation, so the set also runs as the 65
launches a decode step makes (`build_stages`: one skinny launch per stage, each on its own input), with the same
bytes.

The same independent linears also run as one launch (`group_of`, optim/linear_chain.py): one grid over the row
blocks of all 113 linears, every output bitwise equal to its own skinny_mm call with the same waves.

The same linears also run as one dependent launch (`build_chain`, optim/linear_chain.py): stages q|k|v, o,
gate|up, down per layer and the head, each stage's input the unit-RMS renormalisation of the output it depends on
in a decode step (o <- v: attention over one cached position returns v; gate|up <- o; down <- up; the next
layer's q|k|v and the head <- down), or, in the independent variant, a fresh unit-RMS vector per stage with no
waits; and as 65 stream-ordered skinny launches with the same dependencies (`stage_graph_calls`: each launch
renormalises its producer's output inside the launch).

Used by bench.py and by `python -m byteprof_amd.profiling`.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass

import torch

from .optim import skinny as S
from .optim.linear_chain import ChainStage, LinearChain
from .quant.accounting import Linear, call_bytes
from .quant.hip_int8 import quantize_rowwise_int8

LAYERS = 16
CHAIN_RB, CHAIN_WAVES = 0, 8  # one-launch set: 8-row blocks per workgroup (0: per linear) and waves per workgroup
HIDDEN, FFN, VOCAB = 2048, 8192, 100352
LAYER_LINEARS = (("q", HIDDEN, HIDDEN), ("k", HIDDEN, HIDDEN), ("v", HIDDEN, HIDDEN), ("o", HIDDEN, HIDDEN),
                 ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN), ("down", HIDDEN, FFN))


def shapes() -> list[tuple[str, int, int]]:
    """(name, N, K) of the 113 linears in decode order."""
    out = [(f"l{layer}.{name}", n, k) for layer in range(LAYERS) for name, n, k in LAYER_LINEARS]
    out.append(("lm_head", VOCAB, HIDDEN))
    return out


def unit_rms(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (xf / xf.pow(2).mean(dim=-1, keepdim=True).sqrt()).to(torch.bfloat16)


@dataclass
class Op:
    name: str
    n: int
    k: int
    args: tuple  # (w,) for bf16, (q, scale) for int8
    x: torch.Tensor
    y: torch.Tensor

    def __call__(self) -> None:
        S.skinny_mm(self.x, *self.args, out=self.y)


def build(kind: str = "bf16", m: int = 1, device="cuda:0", seed: int = 0, scale_dtype=torch.float16,
          weights: dict | None = None) -> list[Op]:
    """Seeded operands of the set; kind 'bf16' or 'int8' (per-row scales in `scale_dtype`). With `weights`
    (make_weights of the same kind) the launches use those tensors and only the inputs are drawn here."""
    g = torch.Generator(device=device).manual_seed(seed)
    ops = []
    for name, n, k in shapes():
        if weights is not None:
            args = weights[name]
        else:
            w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
            args = (w,) if kind == "bf16" else quantize_rowwise_int8(w, scale_dtype)
            del w
        x = unit_rms(torch.randn(m, k, generator=g, device=device))
        ops.append(Op(name, n, k, args, x, torch.empty(m, n, dtype=torch.bfloat16, device=device)))
    return ops


def group_of(ops: list[Op], rb: int = CHAIN_RB, waves: int = CHAIN_WAVES) -> LinearChain:
    """The ops (each on its own input, M = 1) as one launch of independent stages writing the ops' own outputs."""
    stages = [ChainStage([o.args if len(o.args) > 1 else o.args[0]], o.x[0], o.y[0]) for o in ops]
    return LinearChain(stages, rb=rb, waves=waves)


def algorithmic_bytes(ops: list[Op], kind: str, m: int) -> int:
    scheme = None if kind == "bf16" else "int8_wo"
    return int(sum(call_bytes(Linear(op.n, op.k), scheme, m) for op in ops))


def capture(calls) -> torch.cuda.CUDAGraph:
    """One HIP graph holding the calls in order (after one warm-up pass on a side stream)."""
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


def time_replays(g: torch.cuda.CUDAGraph, replays: int, trials: int) -> list[float]:
    """ms per replay for each trial, from HIP events on the stream the replays run on."""
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


def dispatch_gap_us(launches: int = 100) -> float:
    """us per launch of an empty kernel (torch.cuda._sleep(0)) back to back in a HIP graph: the fixed cost a
    dependent launch adds on this device."""
    g = capture([lambda: torch.cuda._sleep(0)] * launches)
    time_replays(g, 2, 1)
    return statistics.median(time_replays(g, 10, 5)) * 1000.0 / launches


def kernel_key(kind: str, n: int, k: int, m: int) -> str:
    """Name of the kernel instantiation a launch uses, as the profiler reports it."""
    return S.kernel_name(kind, n, k, m)


# stages of one layer: (stage name, linears sharing its input)
LAYER_STAGES = (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gateup", ("gate", "up")), ("down", ("down",)))


@dataclass
class Chain:
    """The decode-step set as the stages of one launch."""

    kind: str
    stages: list
    lset: LinearChain
    weights: dict  # linear name -> (w,) or (q, scale)


def make_weights(kind: str = "bf16", device="cuda:0", seed: int = 0, scale_dtype=torch.float16) -> dict:
    """Seeded weights of the 113 linears, keyed by name (l{layer}.{q,k,v,o,gate,up,down}, lm_head). The linears of
    one stage are adjacent rows of one allocation, also keyed by the stage (l{layer}.qkv = q|k|v, l{layer}.gateup =
    gate|up), so a stage can run as one launch; per-row int8 scales make the two views quantise alike."""
    g = torch.Generator(device=device).manual_seed(seed)
    out = {}

    def add(key, names_rows, k):
        w = (torch.randn(sum(n for _, n in names_rows), k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        full = (w,) if kind == "bf16" else quantize_rowwise_int8(w, scale_dtype)
        del w
        out[key] = full
        r = 0
        for name, n in names_rows:
            out[name] = tuple(t[r:r + n] for t in full)
            r += n

    for layer in range(LAYERS):
        pre = f"l{layer}."
        for stage, names in LAYER_STAGES:
            dims = {nm: (n, k) for nm, n, k in LAYER_LINEARS}
            add(pre + stage, [(pre + nm, dims[nm][0]) for nm in names], dims[names[0]][1])
    add("lm_head", [("lm_head", VOCAB)], HIDDEN)
    return out


def stage_keys() -> list[str]:
    """Keys of the 65 stages' weights in decode order (make_weights)."""
    return [f"l{layer}.{stage}" for layer in range(LAYERS) for stage, _ in LAYER_STAGES] + ["lm_head"]


def stage_shapes() -> list[tuple[str, int, int]]:
    """(key, N, K) of the 65 stages in decode order: q|k|v 6144 x 2048, o 2048 x 2048, gate|up 16384 x 2048, down
    2048 x 8192 per layer, then the LM head."""
    dims = {nm: (n, k) for nm, n, k in LAYER_LINEARS}
    out = []
    for layer in range(LAYERS):
        for stage, names in LAYER_STAGES:
            out.append((f"l{layer}.{stage}", sum(dims[nm][0] for nm in names), dims[names[0]][1]))
    out.append(("lm_head", VOCAB, HIDDEN))
    return out


def build_stages(weights: dict, m: int = 1, device="cuda:0", seed: int = 0) -> list[Op]:
    """The set as 65 skinny launches, one per stage over the stage's adjacent weight rows (make_weights), each on
    its own seeded unit-RMS input of m rows: the launches a decode step makes (q|k|v and gate|up share their
    inputs), with the same bytes as the 113 separate linears."""
    g = torch.Generator(device=device).manual_seed(seed)
    ops = []
    for key, n, k in stage_shapes():
        x = unit_rms(torch.randn(m, k, generator=g, device=device))
        ops.append(Op(key, n, k, weights[key], x, torch.empty(m, n, dtype=torch.bfloat16, device=device)))
    return ops


def chain_stages(weights: dict, dependent: bool = True, device="cuda:0", seed: int = 1) -> list:
    """Stages of the set in decode order over `weights` (make_weights). dependent: each stage reads (renormalised)
    the output it depends on in a decode step; otherwise each stage has its own unit-RMS input and no wait."""
    g = torch.Generator(device=device).manual_seed(seed)

    def fresh(k):
        return unit_rms(torch.randn(1, k, generator=g, device=device))[0].contiguous()

    stages: list = []
    prev = None  # stage index feeding the next qkv / head

    def add(names, src, renorm):
        ws = [weights[nm] if len(weights[nm]) > 1 else weights[nm][0] for nm in names]
        n = sum(int((w[0] if isinstance(w, tuple) else w).shape[0]) for w in ws)
        stages.append(ChainStage(ws, src, torch.empty(n, dtype=torch.bfloat16, device=device), renorm))
        return len(stages) - 1

    for layer in range(LAYERS):
        pre = f"l{layer}."
        if not dependent:
            for _, names in LAYER_STAGES:
                k = int(weights[pre + names[0]][0].shape[1])
                add([pre + nm for nm in names], fresh(k), False)
            continue
        i_qkv = add([pre + "q", pre + "k", pre + "v"], fresh(HIDDEN) if prev is None else (prev, 0), True)
        i_o = add([pre + "o"], (i_qkv, 2 * HIDDEN), True)
        i_gu = add([pre + "gate", pre + "up"], (i_o, 0), True)
        prev = add([pre + "down"], (i_gu, FFN), True)
    if dependent:
        add(["lm_head"], (prev, 0), True)
    else:
        add(["lm_head"], fresh(HIDDEN), False)
    return stages


def build_chain(kind: str = "bf16", device="cuda:0", seed: int = 0, scale_dtype=torch.float16,
                dependent: bool = True, weights: dict | None = None, rb: int = CHAIN_RB,
                waves: int = CHAIN_WAVES) -> Chain:
    """The set as one launch (weights from make_weights unless given)."""
    weights = weights if weights is not None else make_weights(kind, device, seed, scale_dtype)
    stages = chain_stages(weights, dependent, device, seed + 1)
    return Chain(kind, stages, LinearChain(stages, rb=rb, waves=waves), weights)


def stage_launches(chain: Chain, rb: int = CHAIN_RB, waves: int = CHAIN_WAVES) -> list[LinearChain]:
    """The dependent set as one launch per stage (65 stream-ordered launches): stage s is a launch of its own linears
    on the renormalised slice of stage s-1's output, read as an ordinary input once the launch before it has
    finished. Same weights and outputs as `chain` (whose stages must be dependent)."""
    out = []
    for st in chain.stages:
        if isinstance(st.src, tuple):
            dep, start = st.src
            k = int((st.weights[0][0] if isinstance(st.weights[0], tuple) else st.weights[0]).shape[1])
            src = chain.stages[dep].out[start:start + k]
        else:
            src = st.src
        out.append(LinearChain([ChainStage(st.weights, src, st.out, st.renorm)], rb=rb, waves=waves))
    return out


def stage_graph_calls(chain: Chain) -> list:
    """The set as 65 stream-ordered launches of the matrix-core skinny kernel, one per stage over the stage's weight
    rows (q|k|v, o, gate|up, down, the head), each reading its input as `chain` defines it: a dependent stage reads
    the slice of its producer's output and renormalises it to unit RMS inside the launch (BP_PRO_UNIT_RMS), so the
    data dependencies of a decode step hold; an independent stage reads its own vector."""
    calls = []
    for key, st in zip(stage_keys(), chain.stages):
        w = chain.weights[key]
        q, scale = (w[0], None) if len(w) == 1 else w
        k = int(q.shape[1])
        if isinstance(st.src, tuple):
            dep, start = st.src
            src = chain.stages[dep].out[start:start + k]
        else:
            src = st.src
        x, y = src.view(1, k), st.out.view(1, -1)
        if st.renorm:
            calls.append(lambda x=x, q=q, scale=scale, y=y: S.prologue_mm(x, q, scale, y, S.PRO_UNIT_RMS))
        else:
            calls.append(lambda x=x, w=w, y=y: S.skinny_mm(x, *w, out=y))
    return calls


def chain_bytes(kind: str) -> int:
    """Algorithmic bytes of one pass of the set at M = 1 (every linear's weights, scales, input and output once;
    the same total as the per-launch set)."""
    scheme = None if kind == "bf16" else "int8_wo"
    return int(sum(call_bytes(Linear(n, k), scheme, 1) for _, n, k in shapes()))
