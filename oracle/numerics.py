"""Rounding and error metrics of the oracle (test infrastructure only; see oracle/__init__.py).

bf16 rounding is done on the fp32 bit pattern with integer arithmetic (round to nearest, ties to even, NaN kept a
quiet NaN), the rule torch's `.to(torch.bfloat16)` and the kernels' v_cvt_pk_bf16_f32 follow. Pinned by known-answer
bit patterns computed by hand in tests/test_oracle.py (ties, carries into the exponent, overflow to inf, NaN,
negative zero, subnormals) and by exhaustive agreement with an exact rational rounding on sampled patterns.
"""

from __future__ import annotations

import numpy as np


def bf16_bits(a) -> np.ndarray:
    """uint16 bf16 patterns of float values (rounded to nearest even)."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint32) & 0xFFFF
    out = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32) & 0xFFFF, out)
    return out.astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    """float32 values of uint16 bf16 patterns (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def bf16_round(a) -> np.ndarray:
    """Values rounded to bf16, returned as float32 (exactly representable)."""
    return from_bf16_bits(bf16_bits(a))


def f16_round(a) -> np.ndarray:
    """Values rounded to IEEE binary16 (numpy's conversion rounds to nearest even), returned as float32."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def io_round(a, io: str) -> np.ndarray:
    """Round to the io dtype ('bf16', 'f16' or 'f32'), returned as float64 (exact)."""
    if io == "bf16":
        return bf16_round(a).astype(np.float64)
    if io == "f16":
        return f16_round(a).astype(np.float64)
    if io == "f32":
        return np.asarray(a, dtype=np.float32).astype(np.float64)
    raise ValueError(io)


def componentwise_error(y, x, w) -> float:
    """max_ij |y - x w^T|_ij / (|x| |w|^T)_ij, the skinny tolerance metric of the reference
    (tests/test_skinny.py:34-40): normalising by the sum of absolute terms keeps cancelling outputs from dominating."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    ref = x @ w.T
    scale = np.maximum(np.abs(x) @ np.abs(w).T, 1e-30)
    return float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref) / scale)) if ref.size else 0.0


def normwise_error(y, ref) -> float:
    """max |y - ref| / max |ref| (tests/test_fused_kernels_gpu.py:37-39; the 1e-2 gate of the decode path)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    return float(np.max(np.abs(y - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
