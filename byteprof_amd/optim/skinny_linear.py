"""`SkinnyLinear`: an `nn.Linear` replacement on the gfx950 skinny kernels (byteprof/optim/skinny_linear.py:20-71).

Schemes bf16_wo (the layer's own bf16 weights), int8_wo (per-row symmetric int8, the quantization `Int8Linear`
uses) and int4_wo (the group-128 tile-major format of `skinny.quantize_int4`). The kernel takes every input of
1..MAX_M bf16 rows on the GPU -- one family of kernels whose rows do not depend on how many share a call --;
an empty input returns an empty output; larger inputs and other dtypes go through `F.linear` on the weights
dequantized (fp32, then the activation dtype) for that call.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import skinny
from .weight_only import WeightOnlyLinear

SCHEMES = {"bf16_wo": "bf16", "int8_wo": "int8", "int4_wo": "int4"}


class SkinnyLinear(WeightOnlyLinear):
    empty_returns_empty = True

    def __init__(self, lin: nn.Linear, scheme: str, tile_rows: int | None = None):
        """tile_rows: int4_wo's row tiles (16, 32 or 64; the reference packs 32); None picks the tuned tile rows
        of the weight's shape (skinny.int4_tile_rows)."""
        if scheme not in SCHEMES:
            raise ValueError(f"unknown scheme {scheme!r}")
        if tile_rows is not None and tile_rows not in skinny.INT4_TILES:
            raise ValueError(f"int4 tile rows must be one of {skinny.INT4_TILES}, got {tile_rows}")
        super().__init__(lin, SCHEMES[scheme], tile_rows)
        self.scheme = scheme

    def _kind(self) -> str:
        return self.kind

    def _kernel_takes(self, x2: torch.Tensor) -> bool:
        return x2.is_cuda and x2.dtype == torch.bfloat16 and 1 <= x2.shape[0] <= skinny.MAX_M

    def _kernel(self, x2: torch.Tensor) -> torch.Tensor:
        return skinny.skinny_mm(x2, *self.operands())

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, {self.scheme}, skinny kernel (gfx950)"
