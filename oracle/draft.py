"""Drafting-round bookkeeping oracle (test infrastructure only; see oracle/__init__.py).

accepted_length: the number of leading drafts ids[1 + j] equal to tok[j], j < S - 1
    (byteprof/optim/mlstm_multistep.py:136-146, draft_core.py:30-37). Pinned by the reference's own known answers
    (tests/test_fused_kernels_gpu.py:116-126, restated as data in tests/test_oracle.py) and the bounds 0 <= L <= S-1.
committed_state: the state after positions 0 .. L of a verify round = oracle.mlstm.multistep over the first L + 1
    positions from the start state (byteprof/optim/mlstm_multistep.py:89-134); L is clamped to the positions given.
    Pinned through oracle.mlstm.multistep (composition, closed forms; tests/test_oracle.py).
"""

from __future__ import annotations

from . import mlstm as OM


def accepted_length(ids, tok, s: int) -> int:
    n = 0
    for j in range(s - 1):
        if int(ids[1 + j]) != int(tok[j]):
            break
        n += 1
    return n


def committed_state(c, n, m, k, v, i, f, length: int, io: str):
    """(c, n, m) float64 after positions 0 .. length (clamped to [-1, T - 1]) from the start state."""
    t = min(max(int(length) + 1, 0), k.shape[0])
    if t == 0:
        import numpy as np

        return np.array(c, dtype=np.float64), np.array(n, dtype=np.float64), np.array(m, dtype=np.float64)
    _, st = OM.multistep(c, n, m, k[:t], k[:t], v[:t], i[:t], f[:t], eps=1e-6, io=io)
    return st
