"""Shared pieces of the GPU tests: seeded inputs and the oracle comparisons (numpy oracle for small and mid sizes;
the reference's own fp32 formulation `x.float() @ dequantize(...).T` for the full-size checks)."""

from __future__ import annotations

import numpy as np
import torch

from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import numerics as ON
from oracle import skinny as OS

TOL_COMPONENTWISE = 4e-3  # byteprof tests/test_skinny.py:17
TOL_NORMWISE = 1e-2  # the bf16 max relative error gate; byteprof tests/test_quant_int8.py:53-56


def make_weights(kind: str, n: int, k: int, seed: int = 0, device: str = "cuda", scale_dtype=None, std=0.02):
    g = torch.Generator(device=device).manual_seed(seed)
    w = (torch.randn(n, k, generator=g, device=device) * std).to(torch.bfloat16)
    if kind == "bf16":
        return w, (w,)
    q, s = quantize_rowwise_int8(w, scale_dtype)
    return w, (q, s)


def oracle_weights(kind: str, args) -> np.ndarray:
    """float32 numpy weights [N, K] the kernel must reproduce (bf16 values or q * scale)."""
    if kind == "bf16":
        return args[0].float().cpu().numpy()
    q, s = args
    return OS.dequantize("int8", q.cpu().numpy(), s.float().cpu().numpy())


def randn_x(m: int, k: int, seed: int, device: str = "cuda") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)


def check_against_oracle(y: torch.Tensor, x: torch.Tensor, w_np: np.ndarray) -> tuple[float, float]:
    """(componentwise, normwise) errors of y against the oracle; asserts both tolerances."""
    xn = x.float().cpu().numpy()
    yn = y.float().cpu().numpy()
    comp = ON.componentwise_error(yn, xn, w_np)
    norm = ON.normwise_error(yn, OS.matmul(xn, w_np))
    assert comp < TOL_COMPONENTWISE, comp
    assert norm < TOL_NORMWISE, norm
    return comp, norm


def torch_reference(x: torch.Tensor, w_fp32: torch.Tensor) -> torch.Tensor:
    """The reference's own oracle formulation (tests/test_skinny.py:38): fp32 matmul of the stored operands."""
    return x.float() @ w_fp32.T


def normwise(y: torch.Tensor, ref: torch.Tensor) -> float:
    return float((y.float() - ref).abs().max() / ref.abs().max().clamp(min=1e-30))
