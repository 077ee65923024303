"""Stored weight bytes of a linear per scheme (pure), and the algorithmic byte count of a skinny call.

`linear_bytes` restates byteprof/quant/accounting.py:53-64, which defines the "stored bytes" the reference divides
by time to get GB/s (also tools/skinny_bench.py:37-42):
  bf16     2 bytes per weight
  int8_wo  1 byte per weight + one 2-byte scale per output row
  int4_wo  0.5 byte per weight + a 2-byte (scale, zero) pair per group of `group_size` inputs per output row
`call_bytes` adds the activations read and the output written once (the HBM roofline numerator used by the bench).
"""

from __future__ import annotations

from dataclasses import dataclass

BF16 = 2


@dataclass(frozen=True)
class Linear:
    out_features: int
    in_features: int
    group: str | None = None


def linear_bytes(lin: Linear, scheme: str | None, group_size: int = 128) -> float:
    weights = lin.out_features * lin.in_features
    if scheme is None:
        return weights * BF16
    if scheme == "int8_wo":
        return weights + lin.out_features * BF16
    if scheme == "int4_wo":
        if lin.in_features % group_size:
            raise ValueError(f"in_features {lin.in_features} not divisible by group_size {group_size}")
        return weights * 0.5 + lin.out_features * (lin.in_features // group_size) * 2 * BF16
    raise ValueError(f"unknown scheme {scheme!r}")


def call_bytes(lin: Linear, scheme: str | None, m: int, group_size: int = 128) -> float:
    """Weights (+ scales) read once, m bf16 activation rows read once, m bf16 output rows written once."""
    return linear_bytes(lin, scheme, group_size) + BF16 * m * (lin.in_features + lin.out_features)
