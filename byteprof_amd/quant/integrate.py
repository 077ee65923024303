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

from typing import Any, Callable

import torch
import torch.nn as nn

from ..optim.weight_only import WeightOnlyLinear
from .hip_int8 import gemv_int8
from .select import group_of, olmo_should_quantize, should_quantize


class Int8Linear(WeightOnlyLinear):
    """Per-row symmetric int8 weights; one row on the GPU (bf16, fp16 or fp32) goes through the fused int8 product
    (`gemv_int8`), every other input through F.linear on q.to(dtype) * scale.to(dtype) (the reference's
    dequantization in the activation dtype, integrate.py:35-46)."""

    def __init__(self, lin: nn.Linear):
        super().__init__(lin, "int8")

    def dequantized(self, dtype: torch.dtype) -> torch.Tensor:
        return self.q.to(dtype) * self.scale.to(dtype)[:, None]

    def _kernel_takes(self, x2: torch.Tensor) -> bool:
        return x2.shape[0] == 1 and x2.is_cuda and x2.dtype in (torch.bfloat16, torch.float16, torch.float32)

    def _kernel(self, x2: torch.Tensor) -> torch.Tensor:
        return gemv_int8(x2, self.q, self.scale)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, int8 rowwise (gfx950)"


def _is_bolmo(model: nn.Module) -> bool:
    """Bolmo keeps a byte-level local encoder beside the global transformer; OLMo 2 has none."""
    return hasattr(model.model, "local_encoder")


def _maker(kernel: str, scheme: str) -> Callable[[nn.Linear], nn.Module]:
    """The module that replaces a selected nn.Linear under (kernel, scheme), or the reference's refusal."""
    if kernel == "skinny":
        from ..optim.skinny_linear import SkinnyLinear

        return lambda lin: SkinnyLinear(lin, scheme)
    if scheme == "int8_wo":
        return Int8Linear
    if scheme == "int4_wo":
        raise NotImplementedError("the default int4_wo path (torchao tinygemm) is not part of the gfx950 stack")
    raise ValueError(f"unknown scheme {scheme!r}")


def _allocated_mib() -> float:
    return torch.cuda.memory_allocated() / 2**20 if torch.cuda.is_available() else 0.0


def apply_quantization(model: nn.Module, target: str, scheme: str, group_size: int = 128,
                       local_scheme: str | None = None, global_scheme: str | None = None,
                       kernel: str = "default") -> dict[str, Any]:
    """Quantize every linear the target selects; returns statistics (same keys as the reference).

    The plan (module name -> scheme, a Bolmo group's override taking precedence over `scheme`) is made first and
    every scheme in it is resolved to its replacement module before the first swap, so an unknown scheme leaves the
    model untouched."""
    select = should_quantize if _is_bolmo(model) else olmo_should_quantize
    overrides = {"local": local_scheme, "global": global_scheme}
    plan = {name: overrides.get(group_of(name) or "") or scheme
            for name, mod in model.named_modules() if isinstance(mod, nn.Linear) and select(name, target)}
    makers = {sch: _maker(kernel, sch) for sch in dict.fromkeys(plan.values())}
    mem_before = _allocated_mib()
    for name, sch in plan.items():
        holder, _, attr = name.rpartition(".")
        parent = model.get_submodule(holder) if holder else model
        setattr(parent, attr, makers[sch](getattr(parent, attr)))
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    stats: dict[str, Any] = dict(target=target, scheme=scheme, local_scheme=local_scheme, global_scheme=global_scheme)
    stats["group_size"] = group_size if "int4_wo" in makers else None
    stats["n_linears"] = len(plan)
    stats["gpu_mem_before_mib"], stats["gpu_mem_after_mib"] = mem_before, _allocated_mib()
    if kernel != "default":
        stats["kernel"] = kernel
    return stats
