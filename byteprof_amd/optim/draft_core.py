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
