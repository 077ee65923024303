"""Skinny matmul and int8 quantizer oracle (test infrastructure only; see oracle/__init__.py).

matmul:     y = x @ W^T accumulated in float64 from the stored operands (the reference's oracle is
            `x.float() @ dequantize(...).T`, tests/test_skinny.py:34-40; float64 is at least as accurate), then
            rounded to bf16 like the kernel output. Pinned by exact rational arithmetic (fractions.Fraction) on small
            random operands and by hand-computed known answers in tests/test_oracle.py.
dequantize: byteprof/optim/skinny.py:209-217 (bf16 -> value, int8 -> q * scale in float32 as torch computes it).
            Pinned by hand-computed rows.
quantize_rowwise_int8: byteprof/quant/triton_int8.py:50-55 — scale = max|row| / 127 in float32, clamped to 1e-12
            (fp16 scales, which the reference does not have: 2^-24, the smallest fp16 subnormal, so that an all-zero
            row keeps a non-zero scale), rounded to the stored dtype; q = round_half_even(w / stored_scale) in float32, clamped to [-127, 127].
            Pinned by known answers derived with exact rational arithmetic plus float32 rounding of each step
            (tests/golden/make_golden.py), by the reference's own bound (|q * s - w| <= 0.51 s + 1e-3,
            tests/test_quant_int8.py:10-16), and by the invariants |q| <= 127 and q = +-127 at the row maximum.
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_round, f16_round


def matmul(x, w) -> np.ndarray:
    """float64 y = x @ w^T of float operands (already the stored values)."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T


def skinny_bf16(x, w) -> np.ndarray:
    """bf16-rounded output (as float32) of a bf16 skinny call: x [M, K], w [N, K] float values of bf16 data."""
    return bf16_round(matmul(x, w).astype(np.float32))


def dequantize(kind: str, w, scale=None) -> np.ndarray:
    """float32 weights [N, K] of a stored format ('bf16': the values; 'int8': q * scale with scale float values)."""
    if kind == "bf16":
        return np.asarray(w, dtype=np.float32)
    if kind == "int8":
        return np.asarray(w, dtype=np.float32) * np.asarray(scale, dtype=np.float32)[:, None]
    raise ValueError(kind)


def skinny_int8(x, q, scale) -> np.ndarray:
    """bf16-rounded output of an int8 skinny call: sum in float64 of the exact products, times the scale."""
    acc = matmul(x, np.asarray(q, dtype=np.float64))
    return bf16_round((acc * np.asarray(scale, dtype=np.float64)[None, :]).astype(np.float32))


def quantize_rowwise_int8(w, scale_dtype: str = "bf16") -> tuple[np.ndarray, np.ndarray]:
    """(q int8 [N, K], stored scale [N] as float32 values) of float weights w [N, K] (values of bf16 data)."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.max(np.abs(w), axis=1) if w.shape[1] else np.zeros(w.shape[0], np.float32)
    floor = np.float32(2.0 ** -24) if scale_dtype == "f16" else np.float32(1e-12)
    s = np.maximum((amax / np.float32(127.0)).astype(np.float32), floor)
    if scale_dtype == "bf16":
        s = bf16_round(s)
    elif scale_dtype == "f16":
        s = f16_round(s)
    elif scale_dtype != "f32":
        raise ValueError(scale_dtype)
    ratio = (w / s[:, None]).astype(np.float32)
    q = np.clip(np.rint(ratio), -127, 127).astype(np.int8)
    return q, s.astype(np.float32)
