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
int4 (group-128, asymmetric; the tile-major format of byteprof/optim/skinny.py:172-217):
quantize_int4: per row and group of 128 inputs, in float32: scale = max((max - min) / 15, 1e-6) rounded to bf16,
            zero = fp16(-min / scale), code = round_half_even(w / scale + zero) clamped to 0..15
            (skinny.py:172-185). Pinned by a hand-derived group (scale and zero exact, codes with ties to even), by the
            reference's half-step bound (test_skinny.py:56-62) and by codes within 0..15 at the group extremes.
pack_int4 / unpack_int4: codes [N, K] <-> [ceil(N/R), K/128, R, 64], byte j of a row's group = code j | code (j + 64)
            << 4, padding rows zero (skinny.py:188-206). Pinned by the round trip and the reference's layout
            known answer (test_skinny.py:47-53).
skinny_int4: y = x @ ((code - zero) * scale)^T in float64 (exact operands: the kernel's products use the codes,
            zeros and activations exactly), rounded to bf16. Pinned by exact rational arithmetic on a small case.
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


GROUP = 128


def pack_int4(codes, tile_rows: int = 32) -> np.ndarray:
    """uint8 [ceil(N/R), K/128, R, 64] of codes [N, K] (0..15)."""
    q = np.asarray(codes, dtype=np.uint8)
    n, k = q.shape
    tiles = -(-n // tile_rows)
    full = np.zeros((tiles * tile_rows, k), dtype=np.uint8)
    full[:n] = q
    out = np.zeros((tiles, k // GROUP, tile_rows, 64), dtype=np.uint8)
    for t in range(tiles):
        for g in range(k // GROUP):
            for r in range(tile_rows):
                row = full[t * tile_rows + r, g * GROUP:(g + 1) * GROUP]
                out[t, g, r] = row[:64] | (row[64:] << 4)
    return out


def unpack_int4(packed, n: int) -> np.ndarray:
    """codes [N, K] of a packed [T, G, R, 64] array."""
    p = np.asarray(packed, dtype=np.uint8)
    tiles, groups, rows, _ = p.shape
    out = np.zeros((tiles * rows, groups * GROUP), dtype=np.uint8)
    for t in range(tiles):
        for g in range(groups):
            blk = p[t, g]  # [R, 64]
            out[t * rows:(t + 1) * rows, g * GROUP:g * GROUP + 64] = blk & 0xF
            out[t * rows:(t + 1) * rows, g * GROUP + 64:(g + 1) * GROUP] = blk >> 4
    return out[:n]


def quantize_int4(w, tile_rows: int = 32):
    """(packed, scale [K/128, N] as float32 values of bf16, zero [K/128, N] as float32 values of fp16) of float
    weights w [N, K] (values of bf16 data); float32 arithmetic in the order of the reference."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % GROUP:
        raise ValueError("int4 needs K % 128 == 0")
    grp = w.reshape(n, k // GROUP, GROUP)
    lo, hi = grp.min(axis=-1), grp.max(axis=-1)
    scale = bf16_round(np.maximum(((hi - lo) / np.float32(15.0)).astype(np.float32), np.float32(1e-6)))
    zero = f16_round((-lo / scale).astype(np.float32))
    t = (grp / scale[..., None]).astype(np.float32) + zero[..., None]
    codes = np.clip(np.rint(t.astype(np.float32)), 0, 15).astype(np.uint8).reshape(n, k)
    return pack_int4(codes, tile_rows), scale.T.copy(), zero.T.copy()


def dequantize_int4(packed, scale, zero) -> np.ndarray:
    """float64 weights [N, K] = (code - zero) * scale, exactly."""
    scale = np.asarray(scale, dtype=np.float64)
    zero = np.asarray(zero, dtype=np.float64)
    groups, n = scale.shape
    codes = unpack_int4(packed, n).astype(np.float64).reshape(n, groups, GROUP)
    return ((codes - zero.T[..., None]) * scale.T[..., None]).reshape(n, groups * GROUP)


def skinny_int4(x, packed, scale, zero) -> np.ndarray:
    """bf16-rounded output (as float32) of an int4 skinny call."""
    return bf16_round(matmul(x, dequantize_int4(packed, scale, zero)).astype(np.float32))
