"""Independent skinny linears at one activation row as one grouped launch (libbyteprof_amd.so: bp_skinny_group_*).

byteprof's set benchmark runs each linear of a decode step as its own `skinny_mm` call on its own input, the calls
captured in one CUDA graph (tools/skinny_bench.py:45-71 -> byteprof/optim/skinny.py:136-166). Launched one at a
time, the small linears are bound by the fixed cost of each launch and by the tail of each short stream, not by
HBM. `SkinnyGroup` computes the same outputs in one launch: the row blocks of every linear form one grid of
short-lived workgroups (2 rows x 4 waves for bf16), so the weights stream back to back.

Every output is bitwise equal to `skinny_mm(x, w, scale, cfg=(rows, waves, 1))` at one activation row (the same
per-row arithmetic: fp32 accumulation of bf16 products, or of exact int8 -> bf16 pairs with the scale on the fp32
sum, then round to nearest-even bf16). Descriptors are made once, here; `run()` is stream-ordered and allocates
nothing, so it can be captured in a HIP graph.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import torch

from .. import _lib


class BpGroupItem(ctypes.Structure):
    """Mirror of `BpGroupItem` in include/byteprof_amd.h (48 bytes)."""

    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("N", ctypes.c_int64), ("K", ctypes.c_int32), ("block0", ctypes.c_int32)]


assert ctypes.sizeof(BpGroupItem) == 48

LUT_SPAN = 256  # BP_GROUP_LUT_SPAN: workgroups per lookup-table entry
CHUNK = {"bf16": 512, "int8": 1024}  # K granularity: one 1 KiB wave-wide load of one row
_KIND_CODE = {"bf16": 0, "int8": 1}

# Workgroup shape (rows, waves) per weight kind, measured on the decode-step set at one activation row: bf16 2 x 4
# streams the 2.56 GB set at ~7.2 TB/s (2 x 2: -1%, 2 x 1: -3%, 4 x 4: -3%, 1 x 4: -18%); int8 2 x 1 the 1.28 GB set
# at ~7.0 TB/s (4 x 1: -4%, 2 x 2: -17%, 2 x 4: -33%).
DEFAULT_CFG = {"bf16": (2, 4), "int8": (2, 1)}


@dataclass
class GroupItem:
    """One linear y = x . w^T at one activation row: x bf16 [K] (or [1, K]), w bf16 / int8 [N, K], y bf16 [N]
    (or [1, N]); int8 weights take a per-row scale [N] (bf16 / fp16 / fp32, one dtype for the group)."""

    x: torch.Tensor
    w: torch.Tensor
    y: torch.Tensor
    scale: torch.Tensor | None = None


def _row(t: torch.Tensor, length: int, what: str) -> None:
    ok = t.dtype == torch.bfloat16 and t.is_contiguous() and t.numel() == length and (
        t.dim() == 1 or (t.dim() == 2 and t.shape[0] == 1))
    if not ok:
        raise ValueError(f"{what} must be a contiguous bf16 [{length}] (or [1, {length}]) tensor, got {t.dtype} "
                         f"{tuple(t.shape)}")


class SkinnyGroup:
    """Independent linears run by one launch of the grouped skinny kernel on the items' device."""

    def __init__(self, items: Sequence[GroupItem | tuple], cfg: tuple[int, int] | None = None) -> None:
        items = [it if isinstance(it, GroupItem) else GroupItem(*it) for it in items]
        if not items:
            raise ValueError("a group needs at least one linear")
        first = items[0].w
        if first.dtype == torch.bfloat16:
            self.kind = "bf16"
        elif first.dtype == torch.int8:
            self.kind = "int8"
        else:
            raise ValueError(f"unsupported weight dtype {first.dtype}")
        device = first.device
        if device.type != "cuda":
            raise ValueError("the grouped launch runs on a GPU (no CPU path)")
        chunk = CHUNK[self.kind]
        self.scale_dtype = None
        for i, it in enumerate(items):
            w = it.w
            if w.dtype != first.dtype or w.dim() != 2 or not w.is_contiguous():
                raise ValueError(f"item {i}: weights must be contiguous [N, K] {first.dtype} tensors")
            n, k = int(w.shape[0]), int(w.shape[1])
            if k == 0 or k % chunk != 0:
                raise ValueError(f"item {i}: K = {k} must be a positive multiple of {chunk} for {self.kind} weights")
            _row(it.x, k, f"item {i}: x")
            _row(it.y, n, f"item {i}: y")
            if it.x.data_ptr() % 16 or w.data_ptr() % 16:
                raise ValueError(f"item {i}: x and w must be 16-byte aligned")
            if self.kind == "int8":
                s = it.scale
                if s is None or s.dim() != 1 or s.shape[0] != n or not s.is_contiguous():
                    raise ValueError(f"item {i}: int8 weights need a contiguous [N] scale")
                if self.scale_dtype is None:
                    self.scale_dtype = s.dtype
                if s.dtype != self.scale_dtype or s.dtype not in (torch.bfloat16, torch.float16, torch.float32):
                    raise ValueError(f"item {i}: scales must all be one of bf16 / fp16 / fp32")
            elif it.scale is not None:
                raise ValueError(f"item {i}: bf16 weights take no scale")
            for t in (it.x, it.y, it.scale):
                if t is not None and t.device != device:
                    raise ValueError(f"item {i}: all tensors must be on {device}")
        L = _lib.lib()
        self.rows, self.waves = cfg if cfg is not None else DEFAULT_CFG[self.kind]
        if not L.bp_skinny_group_config_supported(_KIND_CODE[self.kind], self.rows, self.waves):
            raise ValueError(f"no compiled grouped kernel for {self.kind} rows={self.rows} waves={self.waves}")
        self.items = items
        self.device = device
        self._host = (BpGroupItem * len(items))()
        for h, it in zip(self._host, items):
            h.x, h.w, h.y = it.x.data_ptr(), it.w.data_ptr(), it.y.data_ptr()
            h.scale = it.scale.data_ptr() if it.scale is not None else None
            h.N, h.K = int(it.w.shape[0]), int(it.w.shape[1])
        total = sum(-(-int(it.w.shape[0]) // self.rows) for it in items)
        lut = (ctypes.c_int32 * max(1, -(-total // LUT_SPAN)))()
        blocks = int(L.bp_skinny_group_plan(ctypes.addressof(self._host), len(items), _KIND_CODE[self.kind],
                                            self.rows, ctypes.addressof(lut), len(lut)))
        if blocks < 0:
            _lib.check(blocks, "bp_skinny_group_plan")
        if blocks != total:
            raise RuntimeError(f"bp_skinny_group_plan returned {blocks} workgroups, expected {total}")
        self.blocks = blocks
        raw = ctypes.string_at(ctypes.addressof(self._host), ctypes.sizeof(self._host))
        self._dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(device)
        self._lut = torch.frombuffer(bytearray(bytes(lut)), dtype=torch.int32).to(device)

    def run(self) -> None:
        """Enqueue one launch on torch's current stream (graph-capturable)."""
        L = _lib.lib()
        scale_dt = _lib.TORCH_DT[self.scale_dtype] if self.scale_dtype is not None else 0
        rc = L.bp_skinny_group_run(_KIND_CODE[self.kind], scale_dt, ctypes.addressof(self._host),
                                   self._dev.data_ptr(), self._lut.data_ptr(), len(self.items), self.blocks,
                                   self.rows, self.waves, _lib.stream_ptr(self.device))
        _lib.check(rc, "bp_skinny_group_run")
