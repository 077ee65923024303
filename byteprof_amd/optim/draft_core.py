"""Device-side pieces of a drafting round's bookkeeping (byteprof/optim/draft_core.py:27-111): the accepted
length of a verify pass and the commit of the accepted position's state from a per-position history, both without a
host read, so that the round can be captured in one graph.
"""

from __future__ import annotations

import torch

from .. import _lib


def accepted_length_t(ids: torch.Tensor, tok: torch.Tensor, s: int) -> torch.Tensor:
    """Accepted length on the device (0-d int32): the number of leading drafts ids[1 + j] equal to tok[j], j < s - 1
    (draft_core.py:35-37)."""
    return torch.cumprod((ids[1:s] == tok[:s - 1]).to(torch.int32), 0).sum()


def commit_state(hist: tuple[torch.Tensor, ...], cur: tuple[torch.Tensor, ...], length: torch.Tensor) -> None:
    """cur <- hist[length] for one layer's state (c, n, m); hist tensors carry a leading slot dimension and length is
    a 0-d integer tensor on the same device (draft_core.py:92-111). On the GPU the slot is read by the kernel (clamped
    to the history); on the CPU it is read on the host, as the reference does."""
    if not cur[0].is_cuda:
        idx = int(length)
        for h, c in zip(hist, cur):
            c.copy_(h[idx])
        return
    c_hist, n_hist, m_hist = hist
    c_cur, n_cur, m_cur = cur
    for h, c in zip(hist, cur):
        if h.dtype != torch.float32 or c.dtype != torch.float32 or not h.is_contiguous() or not c.is_contiguous():
            raise ValueError("commit_state needs contiguous float32 state tensors")
        if h.shape[0] != c_hist.shape[0] or h[0].numel() != c.numel():
            raise ValueError("history slots must match the state shapes")
    if length.numel() != 1 or length.dtype != torch.int64 or length.device != c_cur.device:
        raise ValueError("length must be a one-element int64 tensor on the state's device")
    if n_cur.numel() > c_cur.numel() or m_cur.numel() > c_cur.numel():
        raise ValueError("the n and m states must not be larger than c")
    rc = _lib.lib().bp_draft_commit(c_hist.data_ptr(), c_cur.data_ptr(), n_hist.data_ptr(), n_cur.data_ptr(),
                                    m_hist.data_ptr(), m_cur.data_ptr(), length.data_ptr(), c_hist.shape[0],
                                    c_cur.numel(), n_cur.numel(), m_cur.numel(), _lib.stream_ptr(c_cur.device))
    _lib.check(rc, "bp_draft_commit")


def mlstm_step_into(prev: tuple[torch.Tensor, ...], new: tuple[torch.Tensor, ...], q: torch.Tensor, k: torch.Tensor,
                    v: torch.Tensor, i: torch.Tensor, f: torch.Tensor, h: torch.Tensor, eps: float,
                    bv: int | None = None) -> None:
    """One mLSTM step written into given buffers (byteprof/optim/draft_core.py:114-141, the step kernel the
    per-step drafting path calls per position): from the state prev = (c [1, NH, DQ, DV], n [1, NH, DQ(, 1)],
    m [1, NH, 1]) and q, k [1, NH, DQ], v [1, NH, DV], gate pre-activations i, f [1, NH(, 1)], writes the cell
    output h [1, NH, DV] and the next state into new (same shapes as prev), so each position's state can go to a
    history slot. The arithmetic of one position of the fused multistep (draft_fused.multistep_fw). new must not
    overlap prev. Float32 state, contiguous tensors."""
    from . import draft_fused as F

    bv = bv or F.BV
    c, n, m = prev
    c2, n2, m2 = new
    if q.dim() != 3 or q.shape[0] != 1:
        raise ValueError("q must be [1, NH, DQ]")
    nh, dq, dv = F._geometry(q, v, bv)
    for t in (c, n, m, c2, n2, m2):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("the state tensors must be contiguous float32")
    if c.numel() != nh * dq * dv or n.numel() != nh * dq or m.numel() != nh:
        raise ValueError("prev does not match q / v")
    if c2.numel() != c.numel() or n2.numel() != n.numel() or m2.numel() != m.numel():
        raise ValueError("new must have prev's shapes")
    for a in (c, n, m):
        for b in (c2, n2, m2):
            if a.data_ptr() < b.data_ptr() + b.numel() * 4 and b.data_ptr() < a.data_ptr() + a.numel() * 4:
                raise ValueError("new must not overlap prev")
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype \
            or h.dtype != q.dtype:
        raise ValueError("q, k, v and h must share one float dtype")
    if i.dtype != f.dtype or i.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("i and f must share one float dtype")
    for name, x, count in (("q", q, nh * dq), ("k", k, nh * dq), ("v", v, nh * dv), ("h", h, nh * dv),
                           ("i", i, nh), ("f", f, nh)):
        if x.numel() != count or not x.is_contiguous():
            raise ValueError(f"{name} must be contiguous with {count} elements")
    for x in (n, m, q, k, v, i, f, h, c2, n2, m2):
        if x.device != c.device:
            raise ValueError("all tensors must be on one device")
    if not c.is_cuda:
        raise ValueError("the step kernel runs on the GPU only")
    rc = _lib.lib().bp_mlstm_step(c.data_ptr(), n.data_ptr(), m.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  i.data_ptr(), f.data_ptr(), h.data_ptr(), c2.data_ptr(), n2.data_ptr(),
                                  m2.data_ptr(), nh, dq, dv, _lib.TORCH_DT[q.dtype], _lib.TORCH_DT[i.dtype],
                                  float(dq) ** -0.5, float(eps), bv, _lib.stream_ptr(c.device))
    _lib.check(rc, "bp_mlstm_step")
