"""Decode-step linear set oracle (test infrastructure only; see oracle/__init__.py).

A set launch computes a chain of stages. Stage s takes an input vector x_s: its source (an external vector, or a
slice of an earlier stage's output), renormalised to unit RMS when the stage asks for it; each of its weights then
gives one skinny output row block, y_s = concatenation of bf16(x_s @ W_j^T) (oracle.skinny.skinny_bf16 /
skinny_int8 per row, the reference's one-row arithmetic of byteprof/optim/skinny.py:36-90 at M = 1).

unit_rms:  bf16(src * inv) with inv = 1 / sqrt(mean(src^2)) (inv = 1 for an all-zero src): "activations
           renormalised to unit RMS per layer input" of the decode-step set. The mean square is taken in float64
           here; the kernel accumulates it in float32 in another order, so elements may differ by one bf16 step
           where src * inv falls next to a rounding boundary (the tests allow exactly that).
           Pinned in tests/test_oracle.py by what the formula fixes independently of its code: a constant vector
           maps to all +-1 exactly (catches a missing mean or square root), scaling src by a power of two changes
           nothing (exact in binary arithmetic), the result has mean square 1 within bf16 rounding, zero stays zero.
chain:     the stage loop itself, pinned by a hand-built two-stage case whose second stage reads the first's output
           and by agreement with the per-stage formula.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .numerics import bf16_round
from .skinny import skinny_bf16, skinny_int8


def unit_rms(src) -> np.ndarray:
    """bf16 values (as float32) of src renormalised to unit RMS; src holds bf16 values."""
    x = np.asarray(src, dtype=np.float32)
    ms = float(np.mean(x.astype(np.float64) ** 2)) if x.size else 0.0
    inv = np.float32(1.0 / np.sqrt(ms)) if ms > 0.0 else np.float32(1.0)
    return bf16_round(x * inv)


@dataclass
class OracleStage:
    """weights: list of float32 [n_j, K] values (bf16 weights) or (q int8 [n_j, K], scale float32 [n_j]) pairs;
    src: ('ext', vector) or ('stage', index, start) reading K elements of that stage's output from `start`."""

    weights: list
    src: tuple
    renorm: bool
    kind: str = "bf16"


def stage_output(stage: OracleStage, x) -> np.ndarray:
    """float32 values of the stage's bf16 outputs for input x [K]."""
    x2 = np.asarray(x, dtype=np.float32)[None, :]
    parts = []
    for w in stage.weights:
        if stage.kind == "bf16":
            parts.append(skinny_bf16(x2, w)[0])
        else:
            q, s = w
            parts.append(skinny_int8(x2, q, s)[0])
    return np.concatenate(parts)


def stage_input(stage: OracleStage, outputs: list) -> np.ndarray:
    if stage.src[0] == "ext":
        src = np.asarray(stage.src[1], dtype=np.float32)
    else:
        _, idx, start = stage.src
        k = (stage.weights[0] if stage.kind == "bf16" else stage.weights[0][0]).shape[1]
        src = outputs[idx][start:start + k]
    return unit_rms(src) if stage.renorm else src


def chain(stages: list) -> tuple[list, list]:
    """(inputs, outputs) of every stage, computed in order."""
    xs, ys = [], []
    for st in stages:
        x = stage_input(st, ys)
        xs.append(x)
        ys.append(stage_output(st, x))
    return xs, ys
