"""The OLMo-2-1B-shaped decode-step linear set at M activation rows, as a captured HIP graph of skinny launches.

Per layer (16): q, k, v, o 2048 -> 2048; gate, up 2048 -> 8192; down 8192 -> 2048; then the LM head
2048 -> 100352: 113 linears in decode order, every weight distinct (2.56 GB in bf16, ten times MI355X's 256 MB
Infinity Cache, so nothing is served from cache across replays). Weights ~ N(0, 0.02^2); each linear's input
~ N(0, 1) renormalised to unit RMS. The reference measures the same linears one call each inside a CUDA graph
(byteprof tools/skinny_bench.py:45-71; FINDINGS "OLMo-2 16-block linear set").

Used by bench.py and by `python -m byteprof_amd.profiling`.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass

import torch

from .optim import skinny as S
from .quant.accounting import Linear, call_bytes
from .quant.hip_int8 import quantize_rowwise_int8

LAYERS = 16
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


def build(kind: str = "bf16", m: int = 1, device="cuda:0", seed: int = 0, scale_dtype=torch.float16) -> list[Op]:
    """Seeded operands of the set; kind 'bf16' or 'int8' (per-row scales in `scale_dtype`)."""
    g = torch.Generator(device=device).manual_seed(seed)
    ops = []
    for name, n, k in shapes():
        w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        args = (w,) if kind == "bf16" else quantize_rowwise_int8(w, scale_dtype)
        x = unit_rms(torch.randn(m, k, generator=g, device=device))
        ops.append(Op(name, n, k, args, x, torch.empty(m, n, dtype=torch.bfloat16, device=device)))
        del w
    return ops


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
    """Name of the kernel instantiation a launch uses, as the profiler reports it (template arguments)."""
    rows, waves, _ = S._resolve(kind, n, k, S._bm(m), None)
    return f"skinny_dot_kernel<{0 if kind == 'bf16' else 1}, {S._bm(m)}, {rows}, {waves}, true>"
