"""Fused multi-step mLSTM recurrence of the drafting path on gfx950 (through libbyteprof_amd.so).

Drop-in for byteprof/optim/draft_fused.py:27-40: `multistep_fw(cur, q, k, v, i, f, h, nstart, mstart, eps)` runs
T = q.shape[0] positions from the state `cur` = (c [1, NH, DQ, DV], n [1, NH, DQ], m [1, NH, 1]) without modifying
it, writes the cell outputs into h[:T] (h: [>= T, NH, DV]) and copies the start n, m into nstart [NH, DQ] and
mstart [NH]. The arithmetic is that of byteprof/optim/mlstm_multistep.py:21-86 (logsigmoid forget gate,
stabiliser m, gate activations rounded to the input dtype, fp32 state, state rounded to the input dtype before the
q products, h = q.C / (max(|q.n|, exp(-m)) + eps), qk_scale = DQ ** -0.5).

Geometry: the reference accepts DQ of one or two 64-wide blocks (draft_fused.py:14-24); this kernel takes DQ a
multiple of 64 up to 256 (so also the 256-wide heads of the 4-head configuration) or 384 / 512, and any DV that is a
multiple of the value block BV (4, 8 or 16). Unsupported geometry raises NotImplementedError, as the reference does.

`lazy_commit` (draft_fused.py:43-56) recomputes the state after the accepted positions 0 .. L from the start state
(L a 0-d device integer, so one captured graph serves every accepted length); `accept` (draft_fused.py:57-62)
writes the verified tokens and the accepted length on the device.
"""

from __future__ import annotations

import torch

from .. import _lib

BV = 4  # value columns per workgroup (4, 8 or 16): 4 gives NH x DV / 4 workgroups (256 at 4 heads of 256)


def supported_dq(dq: int) -> bool:
    """Head dims the fused kernel takes: one row of q per thread up to 256 (a multiple of 64), two rows per thread
    at 384 and 512 (workgroups of whole 64-lane waves)."""
    return dq > 0 and dq % 64 == 0 and (dq <= 256 or dq in (384, 512))


def _geometry(q: torch.Tensor, v: torch.Tensor, bv: int) -> tuple[int, int, int]:
    _, nh, dq = q.shape
    dv = v.shape[-1]
    if not supported_dq(dq):
        raise NotImplementedError(f"the fused kernel needs head_dim_qk a multiple of 64 up to 256, or 384 / 512 "
                                  f"(got {dq})")
    if dv % bv:
        raise NotImplementedError(f"head_dim_v {dv} is not a multiple of the value block {bv}")
    return nh, dq, dv


def multistep_fw(cur: tuple[torch.Tensor, ...], q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, i: torch.Tensor,
                 f: torch.Tensor, h: torch.Tensor, nstart: torch.Tensor, mstart: torch.Tensor, eps: float,
                 bv: int | None = None) -> None:
    """T = q.shape[0] positions from the state `cur` (not modified); h (>= T, NH, DV) receives the cell outputs;
    the start n and m are copied to nstart (NH, DQ) and mstart (NH,)."""
    bv = bv or BV
    nh, dq, dv = _geometry(q, v, bv)
    t = q.shape[0]
    c, n, m = cur
    if c.dtype != torch.float32 or n.dtype != torch.float32 or m.dtype != torch.float32:
        raise NotImplementedError("the state must be float32")
    if not (c.is_contiguous() and n.is_contiguous() and m.is_contiguous()):
        raise ValueError("the state tensors must be contiguous")
    if c.numel() != nh * dq * dv or n.numel() != nh * dq or m.numel() != nh:
        raise ValueError("state shapes do not match q / v")
    if q.dtype not in _lib.TORCH_DT or q.dtype == torch.int8 or k.dtype != q.dtype or v.dtype != q.dtype \
            or h.dtype != q.dtype:
        raise ValueError("q, k, v and h must share one float dtype")
    if i.dtype != f.dtype or i.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("i and f must share one float dtype")
    for name, x, inner in (("q", q, (dq, 1)), ("k", k, (dq, 1)), ("v", v, (dv, 1)), ("h", h, (dv, 1))):
        if x.stride()[1:] != inner:
            raise ValueError(f"{name} must be contiguous within a position")
    if k.shape != q.shape or k.stride(0) != q.stride(0) or v.shape[:2] != (t, nh) or h.shape[0] < t:
        raise ValueError("q, k, v, h shapes disagree")
    if i.shape[:2] != (t, nh) or f.shape[:2] != (t, nh) or i.stride(0) != f.stride(0) or \
            (i.dim() == 3 and i.stride(1) != 1) or (i.dim() == 2 and i.stride(1) != 1):
        raise ValueError("i and f must be [T, NH(, 1)] with matching strides")
    if nstart.numel() != nh * dq or mstart.numel() != nh or nstart.dtype != torch.float32 or \
            mstart.dtype != torch.float32 or not nstart.is_contiguous() or not mstart.is_contiguous():
        raise ValueError("nstart / mstart must be contiguous float32 [NH, DQ] / [NH]")
    for x in (q, k, v, i, f, h, nstart, mstart, n, m):
        if x.device != c.device:
            raise ValueError("all tensors must be on one device")
    if not c.is_cuda:
        raise ValueError("the fused kernel runs on the GPU only")
    rc = _lib.lib().bp_mlstm_multistep(
        c.data_ptr(), n.data_ptr(), m.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(),
        f.data_ptr(), h.data_ptr(), nstart.data_ptr(), mstart.data_ptr(), t, nh, dq, dv, q.stride(0), v.stride(0),
        i.stride(0), h.stride(0), _lib.TORCH_DT[q.dtype], _lib.TORCH_DT[i.dtype], float(dq) ** -0.5, float(eps), bv,
        _lib.stream_ptr(c.device))
    _lib.check(rc, "bp_mlstm_multistep")


def _check_state(cur, nh: int, dq: int, dv: int) -> None:
    c, n, m = cur
    if c.dtype != torch.float32 or n.dtype != torch.float32 or m.dtype != torch.float32:
        raise NotImplementedError("the state must be float32")
    if not (c.is_contiguous() and n.is_contiguous() and m.is_contiguous()):
        raise ValueError("the state tensors must be contiguous")
    if c.numel() != nh * dq * dv or n.numel() != nh * dq or m.numel() != nh:
        raise ValueError("state shapes do not match k / v")


def lazy_commit(cur: tuple[torch.Tensor, ...], k: torch.Tensor, v: torch.Tensor, i: torch.Tensor, f: torch.Tensor,
                length: torch.Tensor, nstart: torch.Tensor, mstart: torch.Tensor, bv: int | None = None) -> None:
    """cur <- the state after positions 0 .. L (L = `length`, a 0-d device integer), recomputed from the start state:
    cur[0] must still hold the start C (multistep_fw leaves it untouched) and nstart / mstart the start n, m it
    copied. Positions past k.shape[0] are not applied (L is clamped to the positions available)."""
    bv = bv or BV
    nh, dq, dv = _geometry(k, v, bv)
    t = k.shape[0]
    _check_state(cur, nh, dq, dv)
    c, n, m = cur
    if length.numel() != 1 or length.dtype != torch.int64:
        raise ValueError("length must be a one-element int64 tensor")
    if k.dtype not in (torch.bfloat16, torch.float16, torch.float32) or v.dtype != k.dtype:
        raise ValueError("k and v must share one float dtype")
    if i.dtype != f.dtype or i.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("i and f must share one float dtype")
    if k.stride()[1:] != (dq, 1) or v.stride()[1:] != (dv, 1) or v.shape[:2] != (t, nh):
        raise ValueError("k and v must be [T, NH, D] and contiguous within a position")
    if i.shape[:2] != (t, nh) or f.shape[:2] != (t, nh) or i.stride(0) != f.stride(0):
        raise ValueError("i and f must be [T, NH(, 1)] with matching strides")
    if nstart.numel() != nh * dq or mstart.numel() != nh or nstart.dtype != torch.float32 or \
            mstart.dtype != torch.float32 or not nstart.is_contiguous() or not mstart.is_contiguous():
        raise ValueError("nstart / mstart must be contiguous float32 [NH, DQ] / [NH]")
    for x in (k, v, i, f, nstart, mstart, n, m, length):
        if x.device != c.device:
            raise ValueError("all tensors must be on one device")
    if not c.is_cuda:
        raise ValueError("the fused kernel runs on the GPU only")
    rc = _lib.lib().bp_mlstm_lazy_commit(
        c.data_ptr(), n.data_ptr(), m.data_ptr(), nstart.data_ptr(), mstart.data_ptr(), k.data_ptr(), v.data_ptr(),
        i.data_ptr(), f.data_ptr(), length.data_ptr(), t, nh, dq, dv, k.stride(0), v.stride(0), i.stride(0),
        _lib.TORCH_DT[k.dtype], _lib.TORCH_DT[i.dtype], bv, _lib.stream_ptr(c.device))
    _lib.check(rc, "bp_mlstm_lazy_commit")


def accept(ids: torch.Tensor, tok: torch.Tensor, out: torch.Tensor, s: int, smax: int) -> None:
    """out[:s] <- tok[:s], out[smax] <- the accepted length: the number of leading drafts ids[1 + j] equal to tok[j]
    (j < s - 1), all on the device (mlstm_multistep.py:136-146)."""
    for name, x, need in (("ids", ids, s), ("tok", tok, s), ("out", out, smax + 1)):
        if x.dtype != torch.int64 or not x.is_contiguous() or x.numel() < need:
            raise ValueError(f"{name} must be a contiguous int64 tensor of at least {need} elements")
    if not 0 <= s <= smax:
        raise ValueError("need 0 <= s <= smax")
    if not ids.is_cuda or tok.device != ids.device or out.device != ids.device:
        raise ValueError("ids, tok and out must be on one GPU")
    _lib.check(_lib.lib().bp_draft_accept(ids.data_ptr(), tok.data_ptr(), out.data_ptr(), s, smax,
                                          _lib.stream_ptr(ids.device)), "bp_draft_accept")
