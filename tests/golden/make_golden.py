"""Writes the known-answer fixtures of tests/golden/ with exact rational arithmetic (fractions), independent of the
oracle's numpy code and of torch:

  quantizer_kat.json  rows of bf16-representable weights and the (q, stored scale) the per-row int8 quantizer of
                      byteprof/quant/triton_int8.py:50-55 must produce: scale = fp32(max|w| / 127) clamped to
                      1e-12 (fp16 scales: 2^-24, its smallest subnormal) and rounded to bf16 (or fp16);
                      q = round_half_even(fp32(w / scale)) clamped to +-127.
                      Includes exact half-way ratios (ties to even), an all-zero row (the clamp), a negative row
                      maximum and a scale that bf16 rounding moves.
  skinny_kat.json     small bf16 operands x [M, K], w [N, K] and the exactly rounded bf16 product x w^T (rounded
                      once from the exact rational sum), with ragged K and a cancelling row.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import random
import sys
from fractions import Fraction
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from tests.exact import BF16, FP16, FP32, bf16_bits_exact, exact_round, f32_bits  # noqa: E402


def bf16_value(x: float) -> float:
    """Nearest bf16 value of a Python float (exact)."""
    r = exact_round(Fraction(x), BF16)
    return float(r)


def quantize_row_exact(row: list[float], scale_fmt) -> tuple[list[int], float]:
    amax = max((abs(Fraction(w)) for w in row), default=Fraction(0))
    s = exact_round(amax / 127, FP32)
    floor = Fraction(2) ** -24 if scale_fmt == FP16 else exact_round(Fraction(1e-12), FP32)
    s = max(s, floor)  # fp16: the smallest subnormal, so that an all-zero row keeps a non-zero scale
    s = exact_round(s, scale_fmt)
    q = []
    for w in row:
        ratio = exact_round(Fraction(w) / s, FP32)
        n = int(ratio // 1)
        rem = ratio - n
        if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
            n += 1
        q.append(max(-127, min(127, n)))
    return q, float(s)


def quantizer_cases() -> list[dict]:
    u = 2.0 ** -7
    rows = [
        # amax = 127 * 2^-7: scale exactly 2^-7; ratios 2.5, 3.5, -2.5, 126.5 are ties (to even: 2, 4, -2, 126)
        [2.5 * u, 3.5 * u, -2.5 * u, 126.5 * u, 127 * u, 0.0, -1.0 * u, 0.5 * u],
        # negative maximum: q = -127 there
        [-0.75, 0.25, 0.5, -0.125, 0.0625, 0.3125, -0.6875, 0.1],
        # all zero: scale clamps to 1e-12 (rounded to the stored dtype), q all zero
        [0.0] * 8,
        # a scale that bf16 rounding moves (max/127 is not a bf16 value)
        [0.03125, -0.0117, 0.0205, 0.0007, -0.0301, 0.0155, 0.0001, -0.0043],
    ]
    rng = random.Random(1234)
    for _ in range(4):
        rows.append([rng.gauss(0.0, 0.02) for _ in range(16)])
    cases = []
    for row in rows:
        row = [bf16_value(w) for w in row]
        for name, fmt in (("bf16", BF16), ("f16", FP16)):
            q, s = quantize_row_exact(row, fmt)
            cases.append({"w": row, "scale_dtype": name, "q": q, "scale": s})
    return cases


def skinny_cases() -> list[dict]:
    rng = random.Random(99)
    cases = []
    for m, n, k in ((1, 5, 40), (3, 7, 37), (4, 3, 128), (2, 9, 1)):
        x = [[bf16_value(rng.gauss(0, 1)) for _ in range(k)] for _ in range(m)]
        w = [[bf16_value(rng.gauss(0, 0.02)) for _ in range(k)] for _ in range(n)]
        if n >= 3 and k >= 2:  # a cancelling output: row 2 of w is minus row 1 except its first element
            w[2] = [-v for v in w[1]]
            w[2][0] = bf16_value(w[2][0] + 0.0078125)
        y_bits = []
        for xi in x:
            row_bits = []
            for wj in w:
                exact = sum(Fraction(a) * Fraction(b) for a, b in zip(xi, wj))
                r = exact_round(exact, BF16)
                row_bits.append(f32_bits(float(r)) >> 16 if r != 0 else 0)
            y_bits.append(row_bits)
        cases.append({"m": m, "n": n, "k": k, "x": x, "w": w, "y_bf16_bits": y_bits})
    return cases


def main() -> None:
    (HERE / "quantizer_kat.json").write_text(json.dumps({"cases": quantizer_cases()}, indent=1) + "\n")
    (HERE / "skinny_kat.json").write_text(json.dumps({"cases": skinny_cases()}) + "\n")
    print("wrote", HERE / "quantizer_kat.json", HERE / "skinny_kat.json")


if __name__ == "__main__":
    assert bf16_bits_exact(1.0) == 0x3F80
    main()
