"""Linear layers whose weights live in a weight-only format and are multiplied by the gfx950 skinny kernels.

`WeightOnlyLinear` holds what every such layer shares: the stored format (bf16 rows; int8 rows with one scale per
output row; int4 group-128 tiles with per-group scale and zero), the attributes callers read (`weight` -- the bf16
parameter, or an empty parameter of the same dtype when the bf16 weights are not kept --, the `q` / `scale` /
`zero` buffers, `bias`), and the two ways a call is computed: a kernel call for the row counts the layer's policy
accepts, and otherwise `F.linear` on the weights dequantized for that call. The reference's two layers are two
policies of this base:
  - `SkinnyLinear` (byteprof/optim/skinny_linear.py:20-71): the kernel for 1..MAX_M bf16 rows on the GPU;
    dequantization in fp32, then cast to the activation dtype; an empty input returns an empty output;
  - `Int8Linear` (byteprof/quant/integrate.py:22-49): the kernel for exactly one bf16 row on the GPU;
    dequantization in the activation dtype (q.to(dtype) * scale.to(dtype)).
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import skinny

KINDS = ("bf16", "int8", "int4")


def _stored(kind: str, w: torch.Tensor, tile_rows: int | None = None) -> dict[str, torch.Tensor]:
    """The buffers of a weight-only format for weights w [N, K]; int4 tiles of tile_rows rows (16, 32 or 64: the
    format's row-tile parameter, byteprof/optim/skinny.py:188-198; None: the tuned choice for the shape)."""
    if kind == "int8":
        from ..quant.hip_int8 import quantize_rowwise_int8

        q, scale = quantize_rowwise_int8(w)
        return {"q": q, "scale": scale}
    packed, scale, zero = skinny.quantize_int4(w, tile_rows or skinny.int4_tile_rows(*w.shape))
    return {"q": packed, "scale": scale, "zero": zero}


class WeightOnlyLinear(nn.Module):
    """Base of the weight-only linears. Subclasses decide which calls the kernel takes (`_kernel_takes`), run it
    (`_kernel`) and dequantize for the others (`dequantized`)."""

    empty_returns_empty = False  # an input of zero rows returns an empty output without a call

    def __init__(self, lin: nn.Linear, kind: str, tile_rows: int | None = None):
        super().__init__()
        if kind not in KINDS:
            raise ValueError(f"unknown weight kind {kind!r}")
        self.kind = kind
        self.in_features, self.out_features = lin.in_features, lin.out_features
        self.bias = lin.bias
        if kind == "bf16":
            self.weight = lin.weight
            self.scale = self.zero = None
            return
        src = lin.weight.data
        # callers read weight.dtype (and Bolmo's cache setup reads it); the bf16 weights themselves are not kept
        self.weight = nn.Parameter(src.new_empty(0), requires_grad=False)
        stored = _stored(kind, src, tile_rows)
        for name in ("q", "scale", "zero"):
            if name in stored:
                self.register_buffer(name, stored[name])
            else:
                setattr(self, name, None)

    def operands(self) -> tuple:
        """(w, scale, zero) as skinny_mm takes them."""
        return (self.weight, None, None) if self.kind == "bf16" else (self.q, self.scale, self.zero)

    def dequantized(self, dtype: torch.dtype) -> torch.Tensor:
        if self.kind == "bf16":
            return self.weight
        return skinny.dequantize(self.kind, self.q, self.scale, self.zero).to(dtype)

    def _kernel_takes(self, x2: torch.Tensor) -> bool:
        raise NotImplementedError

    def _kernel(self, x2: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        flat = x.reshape(-1, self.in_features)
        if flat.shape[0] == 0 and self.empty_returns_empty:
            return x.new_empty(*x.shape[:-1], self.out_features)
        if self._kernel_takes(flat):
            y = self._kernel(flat if flat.is_contiguous() else flat.contiguous())
            if self.bias is not None:
                y = y + self.bias
        else:
            y = F.linear(flat, self.dequantized(x.dtype), self.bias)
        return y.reshape(*x.shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, {self.kind} weights (gfx950)"
