"""A decode step's skinny linears as one persistent launch (libbyteprof_amd.so: bp_linear_set_*).

byteprof replays a decode step's linears one `SkinnyLinear.forward` -> `skinny_mm` call each inside a CUDA graph
(byteprof/optim/olmo.py:164-215, byteprof/optim/skinny_linear.py:56-69, byteprof/optim/skinny.py:136-166). At one
activation row every such call is a short weight stream, and on MI355X the fixed cost of a dependent launch is
comparable to streaming a 2048 x 2048 weight. `LinearSet` runs a whole chain of them in one launch: a stage is one
or more linears sharing an input vector (q|k|v, gate|up, o, down, the LM head); a stage can read an earlier stage's
output (the data dependency of a decode step), optionally renormalised to unit RMS; rows are computed exactly as
`skinny_mm` computes them at M = 1 (fp32 accumulation, int8 scale on the fp32 sum, bf16 output).

The launch is stream-ordered and allocation-free (descriptors and scratch are made once, here), so it can be
captured in a HIP graph and replayed; the scratch is never reset (each launch tags its outputs with its own
generation).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from .. import _lib


class BpSetStage(ctypes.Structure):
    """Mirror of `BpSetStage` in include/byteprof_amd.h (128 bytes)."""

    _fields_ = [("src", ctypes.c_void_p), ("y", ctypes.c_void_p), ("x_used", ctypes.c_void_p),
                ("K", ctypes.c_int32), ("N", ctypes.c_int32), ("wait_stage", ctypes.c_int32),
                ("renorm", ctypes.c_int32), ("nseg", ctypes.c_int32), ("seg_end", ctypes.c_int32 * 4),
                ("reserved", ctypes.c_int32), ("w", ctypes.c_void_p * 4), ("scale", ctypes.c_void_p * 4)]


assert ctypes.sizeof(BpSetStage) == 128

MAX_SEGMENTS = 4
ERROR_WORD = 32  # scratch word set by a launch that gave up waiting (include/byteprof_amd.h)
_KIND_CODE = {"bf16": 0, "int8": 1}


@dataclass
class Stage:
    """One stage: `weights` (1..4 tensors [n_j, K], all bf16 or all int8 with `scales`) applied to one input.

    src: bf16 [K] contiguous, the input vector (an external tensor or a slice of an earlier stage's `out`);
    out: bf16 [sum n_j] contiguous, receives the rows of all weights in order;
    wait: index of the earlier stage whose `out` src reads (-1: src is ready before the launch);
    renorm: use bf16(src / rms(src)) instead of src;
    x_used: optional bf16 [K] tensor that receives the input vector the stage used.
    """

    weights: list
    src: torch.Tensor
    out: torch.Tensor
    scales: list | None = None
    wait: int = -1
    renorm: bool = False
    x_used: torch.Tensor | None = None

    @property
    def k(self) -> int:
        return int(self.weights[0].shape[1])

    @property
    def n(self) -> int:
        return int(sum(w.shape[0] for w in self.weights))


def _check_vector(t: torch.Tensor, length: int, what: str) -> None:
    if t.dtype != torch.bfloat16 or t.dim() != 1 or t.shape[0] != length or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous bf16 vector of {length} elements, got {t.dtype} "
                         f"{tuple(t.shape)}")


@dataclass
class LinearSet:
    """A chain of stages run by one launch of the persistent set kernel on `stages[0].src.device`."""

    stages: list
    kind: str = field(init=False)
    scale_dtype: torch.dtype | None = field(init=False, default=None)

    def __post_init__(self) -> None:
        if not self.stages:
            raise ValueError("a linear set needs at least one stage")
        first = self.stages[0].weights[0]
        if first.dtype == torch.bfloat16:
            self.kind = "bf16"
        elif first.dtype == torch.int8:
            self.kind = "int8"
        else:
            raise ValueError(f"unsupported weight dtype {first.dtype}")
        device = self.stages[0].src.device
        chunk = 512 if self.kind == "bf16" else 1024
        for idx, st in enumerate(self.stages):
            if not 1 <= len(st.weights) <= MAX_SEGMENTS:
                raise ValueError(f"stage {idx}: 1..{MAX_SEGMENTS} weights per stage")
            k = st.k
            for w in st.weights:
                if w.dtype != first.dtype or w.dim() != 2 or w.shape[1] != k or not w.is_contiguous():
                    raise ValueError(f"stage {idx}: weights must be contiguous [n, {k}] {first.dtype} tensors")
                if w.device != device:
                    raise ValueError(f"stage {idx}: all tensors must be on {device}")
            if k % chunk != 0:
                raise ValueError(f"stage {idx}: K = {k} must be a multiple of {chunk} for {self.kind} weights")
            if self.kind == "int8":
                if st.scales is None or len(st.scales) != len(st.weights):
                    raise ValueError(f"stage {idx}: int8 weights need one scale vector per weight")
                for w, s in zip(st.weights, st.scales):
                    if s.dim() != 1 or s.shape[0] != w.shape[0] or not s.is_contiguous() or s.device != device:
                        raise ValueError(f"stage {idx}: scales must be contiguous [n] vectors on {device}")
                    if self.scale_dtype is None:
                        self.scale_dtype = s.dtype
                    if s.dtype != self.scale_dtype or s.dtype not in (torch.bfloat16, torch.float16, torch.float32):
                        raise ValueError(f"stage {idx}: scales must all be one of bf16 / fp16 / fp32")
            elif st.scales is not None:
                raise ValueError(f"stage {idx}: bf16 weights take no scales")
            _check_vector(st.src, k, f"stage {idx}: src")
            _check_vector(st.out, st.n, f"stage {idx}: out")
            if st.x_used is not None:
                _check_vector(st.x_used, k, f"stage {idx}: x_used")
            if not -1 <= st.wait < idx:
                raise ValueError(f"stage {idx}: wait must be -1 or an earlier stage, got {st.wait}")
            if st.wait >= 0 and not _inside(st.src, self.stages[st.wait].out):
                raise ValueError(f"stage {idx}: src must lie inside stage {st.wait}'s out")
            for t in (st.src, st.out, st.x_used):
                if t is not None and t.device != device:
                    raise ValueError(f"stage {idx}: all tensors must be on {device}")
        if device.type != "cuda":
            raise ValueError("the linear set runs on a GPU (no CPU path)")
        self.device = device
        L = _lib.lib()
        self.workgroups = int(L.bp_linear_set_workgroups(device.index if device.index is not None else 0))
        if self.workgroups <= 0:
            raise RuntimeError("bp_linear_set_workgroups failed")
        self._host = (BpSetStage * len(self.stages))()
        for h, st in zip(self._host, self.stages):
            h.src, h.y = st.src.data_ptr(), st.out.data_ptr()
            h.x_used = st.x_used.data_ptr() if st.x_used is not None else None
            h.K, h.N, h.wait_stage, h.renorm, h.nseg = st.k, st.n, st.wait, int(st.renorm), len(st.weights)
            end = 0
            for j, w in enumerate(st.weights):
                end += int(w.shape[0])
                h.seg_end[j] = end
                h.w[j] = w.data_ptr()
                if st.scales is not None:
                    h.scale[j] = st.scales[j].data_ptr()
        _lib.check(L.bp_linear_set_validate(ctypes.addressof(self._host), len(self.stages),
                                            _KIND_CODE[self.kind], self.workgroups), "bp_linear_set_validate")
        raw = ctypes.string_at(ctypes.addressof(self._host), ctypes.sizeof(self._host))
        self._dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(device)
        self.scratch_bytes = int(L.bp_linear_set_scratch_bytes(ctypes.addressof(self._host), len(self.stages),
                                                               self.workgroups))
        self.scratch = torch.zeros(self.scratch_bytes // 4, dtype=torch.int32, device=device)

    def run(self) -> None:
        """Enqueue one launch on torch's current stream (graph-capturable)."""
        L = _lib.lib()
        scale_dt = _lib.TORCH_DT[self.scale_dtype] if self.scale_dtype is not None else 0
        rc = L.bp_linear_set_run(_KIND_CODE[self.kind], scale_dt, ctypes.addressof(self._host), self._dev.data_ptr(),
                                 len(self.stages), self.scratch.data_ptr(), self.scratch_bytes, self.workgroups,
                                 _lib.stream_ptr(self.device))
        _lib.check(rc, "bp_linear_set_run")

    def timed_out(self) -> bool:
        """True if a launch since the last clear_error() gave up waiting for another workgroup (synchronises)."""
        return bool(int(self.scratch[ERROR_WORD].item()) != 0)

    def clear_error(self) -> None:
        self.scratch[ERROR_WORD].zero_()


def _inside(t: torch.Tensor, base: torch.Tensor) -> bool:
    lo, hi = base.data_ptr(), base.data_ptr() + base.numel() * base.element_size()
    return lo <= t.data_ptr() and t.data_ptr() + t.numel() * t.element_size() <= hi
