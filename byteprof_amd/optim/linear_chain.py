"""A list of M = 1 linears in one launch of the skinny matrix-core kernel (libbyteprof_amd.so: bp_chain_*).

byteprof runs a decode step's linears one skinny_mm call each inside a CUDA graph (byteprof/optim/olmo.py:164-215,
skinny_linear.py:56-69; its set benchmark, tools/skinny_bench.py:45-71, times the same calls on independent
inputs). On MI355X a dependent launch costs ~1.7 us before it streams anything, about as long as a 2048 x 2048
weight takes to stream. `LinearChain` runs the linears as one grid whose workgroups are ordered by stage:

  - a stage is one or more linears sharing an input vector (q|k|v, o, gate|up, down, the LM head); its input is an
    external vector, or a slice of an earlier stage's output (the data dependency of a decode step), optionally
    renormalised to unit RMS;
  - a workgroup issues its weight loads before it waits for its input, so weights stream across stage boundaries;
  - without dependencies (every stage on an external input) it is the grouped form of the reference's set
    benchmark.

Rows are computed exactly as skinny_mm computes them at M = 1 with the same plan (weight blocks, waves, split 1):
bitwise the same outputs. The launch allocates nothing and is stream-ordered, so it can be captured in a HIP graph
and replayed; its scratch (generation, per-stage counters, error word) is made once here and never reset by the
host.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from .. import _lib


class BpChainItem(ctypes.Structure):
    """Mirror of `BpChainItem` in include/byteprof_amd.h (88 bytes)."""

    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("tag_out", ctypes.c_void_p), ("tag_in", ctypes.c_void_p), ("n", ctypes.c_int64),
                ("K", ctypes.c_int64), ("first_wg", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("stage", ctypes.c_int32), ("dep_stage", ctypes.c_int32), ("dep_wgs", ctypes.c_int32),
                ("rb", ctypes.c_int32)]


assert ctypes.sizeof(BpChainItem) == 88

RENORM = 1  # BP_CHAIN_RENORM
ERROR_WORD = 2
_KIND_CODE = {"bf16": 0, "int8": 1}


@dataclass
class ChainStage:
    """One stage: `weights` (tensors [n_j, K], all bf16, or all (q int8, scale) pairs) applied to one input.

    src: a bf16 [K] tensor (external input), or (stage index, start): K elements of that earlier stage's output from
         `start`;
    out: bf16 [sum n_j] contiguous, receives the rows of all weights in order;
    renorm: use bf16(v / sqrt(mean(v^2))) of the source instead of the source itself."""

    weights: list
    src: object
    out: torch.Tensor
    renorm: bool = False


class LinearChain:
    """The stages as one launch. rb: 8-row blocks per workgroup for every item (1, 2, 4), or 0: per item, the most
    blocks whose whole weight tile is in flight before the input wait. waves: per workgroup (2, 4, 8); the K order
    of every row (its outputs equal skinny_mm's with the same waves and split 1)."""

    def __init__(self, stages: list[ChainStage], rb: int = 0, waves: int = 8):
        if not stages:
            raise ValueError("no stages")
        first = stages[0].weights[0]
        self.kind = "int8" if isinstance(first, tuple) else "bf16"
        self.stages, self.rb, self.waves = stages, rb, waves
        L = _lib.lib()
        kc = _KIND_CODE[self.kind]
        if not L.bp_chain_supported(kc, rb, waves):
            raise ValueError(f"no chain kernel for {self.kind} with rb={rb}, waves={waves}")
        dev = stages[0].out.device
        consumed = {st.src[0] for st in stages if isinstance(st.src, tuple)}
        self.dependent = bool(consumed)
        for i, st in enumerate(stages):
            if isinstance(st.src, tuple) and not 0 <= st.src[0] < i:
                raise ValueError(f"stage {i} reads stage {st.src[0]}, which does not come before it")
        # tagged copies of the outputs other stages read
        self.tagged = {i: torch.zeros(stages[i].out.numel(), dtype=torch.int32, device=dev) for i in consumed}
        self.scale_dtype = None
        items = []
        keep = []
        for i, st in enumerate(stages):
            off = 0
            for w in st.weights:
                q, sc = (w if isinstance(w, tuple) else (w, None))
                if (sc is None) != (self.kind == "bf16"):
                    raise ValueError("all stages must hold the same weight kind")
                if sc is not None:
                    if self.scale_dtype is None:
                        self.scale_dtype = sc.dtype
                    elif sc.dtype != self.scale_dtype:
                        raise ValueError("all int8 scales must have one dtype")
                n, k = int(q.shape[0]), int(q.shape[1])
                it = BpChainItem()
                it.w, it.scale = q.data_ptr(), (sc.data_ptr() if sc is not None else None)
                it.y = st.out.data_ptr() + 2 * off
                it.tag_out = self.tagged[i].data_ptr() + 4 * off if i in self.tagged else None
                if isinstance(st.src, tuple):
                    dep, start = st.src
                    if start < 0 or start + k > stages[dep].out.numel() or start % 2:
                        raise ValueError(f"stage {i}: the slice of stage {dep}'s output must start at an even "
                                         "index and end inside it")
                    it.x, it.tag_in = None, self.tagged[dep].data_ptr() + 4 * start
                    it.dep_stage = dep
                else:
                    if (st.src.numel() != k or not st.src.is_contiguous() or st.src.dtype != torch.bfloat16
                            or st.src.data_ptr() % 8):
                        raise ValueError(f"stage {i}: the input must be a contiguous, 8-byte aligned bf16 [{k}] tensor")
                    it.x, it.tag_in, it.dep_stage = st.src.data_ptr(), None, -1
                    keep.append(st.src)
                it.n, it.K, it.stage = n, k, i
                it.flags = RENORM if st.renorm else 0
                items.append(it)
                off += n
            if off != st.out.numel():
                raise ValueError(f"stage {i}: out holds {st.out.numel()} rows, the weights {off}")
        arr = (BpChainItem * len(items))(*items)
        total = L.bp_chain_plan(arr, len(items), kc, rb, waves, None, 0)
        if total < 0:
            _lib.check(total, "bp_chain_plan")
        lut = (ctypes.c_int32 * (-(-total // 256)))()
        _lib.check(min(0, L.bp_chain_plan(arr, len(items), kc, rb, waves, lut, len(lut))), "bp_chain_plan")
        self.stage_wgs: dict[int, int] = {}
        for it in arr:
            self.stage_wgs[it.stage] = self.stage_wgs.get(it.stage, 0) + -(-it.n // (8 * it.rb))
        self.total_wgs = total
        self.items = torch.frombuffer(bytearray(arr), dtype=torch.uint8).to(dev)
        self.lut = torch.tensor(list(lut), dtype=torch.int32, device=dev)
        self.scratch = torch.zeros(-(-L.bp_chain_scratch_bytes(len(stages)) // 4), dtype=torch.int32, device=dev)
        self._keep = keep
        self.n_items = len(items)

    def run(self) -> None:
        """One launch on torch's current stream."""
        L = _lib.lib()
        sdt = _lib.TORCH_DT[self.scale_dtype] if self.scale_dtype is not None else 0
        rc = L.bp_chain_run(_KIND_CODE[self.kind], sdt, self.items.data_ptr(), self.lut.data_ptr(), self.n_items,
                            self.total_wgs, self.waves, self.scratch.data_ptr(), int(self.dependent),
                            _lib.stream_ptr(self.items.device))
        _lib.check(rc, "bp_chain_run")

    def timed_out(self) -> bool:
        """Whether a launch gave up waiting (its outputs are then invalid); reads the scratch (synchronises)."""
        return bool(int(self.scratch[ERROR_WORD].item()))
