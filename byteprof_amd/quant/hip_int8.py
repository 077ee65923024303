"""Fused int8 weight-only products on gfx950 and the per-row int8 quantizer.

Drop-in for byteprof/quant/triton_int8.py: `gemv_int8(x, w, scale, cfg=None, out=None)` computes
y[1, n] = scale[n] * sum_k float(w[n, k]) * float(x[k]) with the int8 -> bf16 conversion fused into the weight
stream (triton_int8.py:16-47); `quantize_rowwise_int8(w)` is the symmetric per-row quantizer (triton_int8.py:50-55),
restated in torch so its bytes are those of the reference.

The product runs on the one-row launch of the skinny matrix-core kernel (the same instructions and K order as
skinny_mm on int8 weights, so the two agree bit for bit). `cfg` is (rows, waves) or the reference's (BN, BK,
num_warps); like the reference, gemv_int8 validates only what raw-pointer kernels need (one row, shapes that agree,
GPU tensors).
"""

from __future__ import annotations

import torch

from .. import _lib
from ..optim import skinny

_X_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
DEFAULT_CFG = None  # chosen per shape by byteprof_amd.optim.skinny.get_cfg (tuned table / heuristic)


def default_cfg(n_out: int, k: int = 2048) -> tuple[int, int]:
    rows, waves, _ = skinny.get_cfg("int8", n_out, k, 1)
    return rows, waves


def gemv_int8(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, cfg: tuple[int, ...] | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """x: [1, K] bf16 / fp16 / fp32, w: [N, K] int8, scale: [N] (bf16 / fp16 / fp32) -> [1, N] in x's dtype.

    The kernel's activation operands are bf16: an fp16 or fp32 row is rounded to bf16 on the way in (the
    reference's GEMV reads x as fp32, triton_int8.py:24; the rounding adds at most 2^-9 of |x| . |w| per output,
    inside the skinny gates) and the bf16 result is cast to x's dtype, as the reference returns it."""
    N, K = w.shape
    if x.numel() != K or not x.is_contiguous() or x.dtype not in _X_DTYPES or not x.is_cuda:
        raise ValueError("x must be a contiguous [1, K] bfloat16, float16 or float32 GPU tensor")
    if not w.is_contiguous() or scale.shape != (N,) or not scale.is_contiguous():
        raise ValueError("w must be a contiguous [N, K] int8 tensor and scale a contiguous [N] tensor")
    y = out if out is not None else torch.empty(1, N, dtype=x.dtype, device=x.device)
    if N == 0:
        return y
    if K == 0:
        y.zero_()
        return y
    if cfg is not None:  # (rows, waves) or (BN, BK, num_warps): the split stays the shape's own (its K order)
        split = skinny.get_cfg("int8", N, K, 1)[2]
        cfg = (int(cfg[0]), int(cfg[-1] if len(cfg) == 2 else cfg[2]), split)
    bf = x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16
    yb = y if bf else torch.empty(1, N, dtype=torch.bfloat16, device=x.device)
    skinny._launch("int8", x.reshape(1, K).to(torch.bfloat16), w, scale, yb, cfg)
    if not bf:
        y.copy_(yb.view_as(y))
    return y


def quantize_rowwise_int8(w: torch.Tensor, scale_dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-output-row int8: w ~ q * scale[:, None], scale stored in `scale_dtype` (default: w.dtype, as in
    the reference; fp16 is the other 2-byte option).

    The scale is rounded to the stored dtype first and q is computed against that stored value; torch.round is
    round-half-to-even (triton_int8.py:50-55)."""
    sdt = scale_dtype or w.dtype
    floor = 2.0 ** -24 if sdt == torch.float16 else 1e-12  # fp16: its smallest subnormal, never a zero scale
    scale = (w.float().abs().amax(dim=1) / 127.0).clamp_min(floor).to(sdt)
    q = torch.round(w.float() / scale.float()[:, None]).clamp_(-127, 127).to(torch.int8)
    return q.contiguous(), scale
