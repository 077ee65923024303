"""Drop-in replacement for an `nn.Linear` that runs the gfx950 skinny kernels (`byteprof_amd.optim.skinny`).

Mirrors byteprof/optim/skinny_linear.py:20-71: schemes bf16_wo (the original bf16 weights) and int8_wo (per-row
symmetric int8, the same quantization as `Int8Linear`); inputs with 1..MAX_M rows on the GPU in bf16 use the
kernel; empty inputs return an empty tensor; larger inputs and non-bf16 activations use the weights dequantized to
the activation dtype with `F.linear`, as the reference does. int4_wo: the skinny group-128 format
(`skinny.quantize_int4`), buffers q (packed), scale and zero, as the reference (skinny_linear.py:39-44).
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import skinny

SCHEMES = ("bf16_wo", "int8_wo", "int4_wo")


class SkinnyLinear(nn.Module):
    def __init__(self, lin: nn.Linear, scheme: str):
        super().__init__()
        if scheme not in SCHEMES:
            raise ValueError(f"unknown scheme {scheme!r}")
        self.scheme = scheme
        self.in_features, self.out_features = lin.in_features, lin.out_features
        self.bias = lin.bias
        w = lin.weight.data
        if scheme == "bf16_wo":
            self.weight = lin.weight  # kept as is: callers read weight.dtype
            self.scale = self.zero = None
            return
        # An empty parameter keeps `weight.dtype` readable without holding the bf16 weights.
        self.weight = nn.Parameter(torch.empty(0, dtype=w.dtype, device=w.device), requires_grad=False)
        if scheme == "int4_wo":
            packed, scale, zero = skinny.quantize_int4(w)
            self.register_buffer("q", packed)
            self.register_buffer("scale", scale)
            self.register_buffer("zero", zero)
            return
        from ..quant.hip_int8 import quantize_rowwise_int8

        q, scale = quantize_rowwise_int8(w)
        self.register_buffer("q", q)
        self.register_buffer("scale", scale)
        self.zero = None

    def _kind(self) -> str:
        return {"bf16_wo": "bf16", "int8_wo": "int8", "int4_wo": "int4"}[self.scheme]

    def dequantized(self, dtype: torch.dtype) -> torch.Tensor:
        if self.scheme == "bf16_wo":
            return self.weight
        return skinny.dequantize(self._kind(), self.q, self.scale, self.zero).to(dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2 = x.reshape(-1, self.in_features)
        if x2.shape[0] == 0:
            return x.new_empty(*x.shape[:-1], self.out_features)
        if x2.is_cuda and x2.dtype == torch.bfloat16 and x2.shape[0] <= skinny.MAX_M:
            if not x2.is_contiguous():
                x2 = x2.contiguous()
            w = self.weight if self.scheme == "bf16_wo" else self.q
            y = skinny.skinny_mm(x2, w, self.scale, self.zero)
            if self.bias is not None:
                y = y + self.bias
        else:
            y = F.linear(x2, self.dequantized(x.dtype), self.bias)
        return y.reshape(*x.shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, {self.scheme}, skinny kernel (gfx950)"
