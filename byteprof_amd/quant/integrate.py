"""Swap a loaded model's selected linears for the gfx950 modules (imported only when a quantization target is set).

Mirrors byteprof/quant/integrate.py:22-122:
  - `Int8Linear(lin)`: per-row symmetric int8 weights; one-row GPU inputs use the fused int8 product
    (`gemv_int8`), every other input the weights dequantized in the activation dtype with F.linear;
  - `apply_quantization(model, target, scheme, group_size=128, local_scheme=None, global_scheme=None,
    kernel="default")`: selects linears by module name (OLMo 2 or Bolmo naming), swaps in `SkinnyLinear` when
    kernel == "skinny", else `Int8Linear` for int8_wo; returns the same statistics dict.
The reference's default int4_wo path is torchao's tinygemm; torchao is not part of this stack, so that branch
raises NotImplementedError.
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn as nn

from ..optim.weight_only import WeightOnlyLinear
from .hip_int8 import gemv_int8
from .select import group_of, olmo_should_quantize, should_quantize


class Int8Linear(WeightOnlyLinear):
    """Per-row symmetric int8 weights; one bf16 row on the GPU goes through the fused int8 product (`gemv_int8`),
    every other input through F.linear on q.to(dtype) * scale.to(dtype) (the reference's dequantization in the
    activation dtype, integrate.py:35-46)."""

    def __init__(self, lin: nn.Linear):
        super().__init__(lin, "int8")

    def dequantized(self, dtype: torch.dtype) -> torch.Tensor:
        return self.q.to(dtype) * self.scale.to(dtype)[:, None]

    def _kernel_takes(self, x2: torch.Tensor) -> bool:
        return x2.shape[0] == 1 and x2.is_cuda and x2.dtype == torch.bfloat16

    def _kernel(self, x2: torch.Tensor) -> torch.Tensor:
        return gemv_int8(x2, self.q, self.scale)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, int8 rowwise (gfx950)"


def _swap(model: nn.Module, name: str, new: nn.Module) -> None:
    parent_name, _, child = name.rpartition(".")
    parent = model.get_submodule(parent_name) if parent_name else model
    setattr(parent, child, new)


def apply_quantization(model: nn.Module, target: str, scheme: str, group_size: int = 128,
                       local_scheme: str | None = None, global_scheme: str | None = None,
                       kernel: str = "default") -> dict[str, Any]:
    """Quantize every linear the target selects; returns statistics (same keys as the reference)."""
    bolmo = hasattr(model.model, "local_encoder")
    pick = should_quantize if bolmo else olmo_should_quantize
    names = [n for n, m in model.named_modules() if isinstance(m, nn.Linear) and pick(n, target)]
    before = torch.cuda.memory_allocated() if torch.cuda.is_available() else 0

    def scheme_of(n: str) -> str:
        g = group_of(n)
        override = local_scheme if g == "local" else global_scheme if g == "global" else None
        return override or scheme

    by_scheme: dict[str, list[str]] = {}
    for n in names:
        by_scheme.setdefault(scheme_of(n), []).append(n)
    for sch, group_names in by_scheme.items():
        if kernel == "skinny":
            from ..optim.skinny_linear import SkinnyLinear

            for n in group_names:
                _swap(model, n, SkinnyLinear(model.get_submodule(n), sch))
        elif sch == "int8_wo":
            for n in group_names:
                _swap(model, n, Int8Linear(model.get_submodule(n)))
        elif sch == "int4_wo":
            raise NotImplementedError("the default int4_wo path (torchao tinygemm) is not part of the gfx950 stack")
        else:
            raise ValueError(f"unknown scheme {sch!r}")
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    after = torch.cuda.memory_allocated() if torch.cuda.is_available() else 0
    stats = {"target": target, "scheme": scheme, "local_scheme": local_scheme, "global_scheme": global_scheme,
             "group_size": group_size if "int4_wo" in by_scheme else None,
             "n_linears": len(names), "gpu_mem_before_mib": before / 2**20, "gpu_mem_after_mib": after / 2**20}
    if kernel != "default":
        stats["kernel"] = kernel
    return stats
