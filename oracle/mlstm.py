"""Multi-step mLSTM recurrence oracle (test infrastructure only; see oracle/__init__.py).

multistep: the stabilised recurrence of byteprof/optim/mlstm_multistep.py:21-86 in float64, with the reference's
    roundings to the io dtype at the points it casts (mlstm_multistep.py:27-29 gate activations; :78-83 state before
    the q products; :85 the stored h). Per position t, per head:
        fl = log(sigmoid(f_t))                          (literal_gate=True: fl = f_t, f read literally as a
                                                          log forget gate, kept only to show the two readings differ)
        m_t = max(fl + m_{t-1}, i_t)
        fa = io(exp(fl + m_{t-1} - m_t)); ia = io(exp(i_t - m_t)); mv = io(exp(-m_t))
        C_t = fa C_{t-1} + ia k_t v_t^T;  n_t = fa n_{t-1} + ia k_t
        h_t = io((qs . io(C_t)) / (max(|qs . io(n_t)|, mv) + eps)),  qs = q_t * qk_scale
    Roundings of the products (k v^T etc.) that the reference's Triton code may apply in bf16 are not reproduced:
    the oracle keeps them exact, which is the more accurate side of the 1e-2 tolerance.
    Pinned by: `unstabilised` below (an independent formula, equal in exact arithmetic when eps = 0 and io = 'f64':
    the stabiliser only rescales C and n by exp(-m_t)); composition (T steps == T1 then T2 steps from the carried
    state); the pure-decay special case i -> -inf; the T = 1 zero-state closed form (h = qs.(k v^T) / max(|qs.k|,
    exp(-i)) when m_0 is very negative). tests/test_oracle.py runs all of them.

unstabilised: C~_t = sigmoid(f_t) C~_{t-1} + exp(i_t) k_t v_t^T, n~ likewise, from C~_0 = C_0 exp(m_0),
    n~_0 = n_0 exp(m_0); h_t = (qs . C~_t) / max(|qs . n~_t|, 1). Only valid where exp does not overflow (small T,
    moderate gates), which is how the tests use it.
"""

from __future__ import annotations

import numpy as np

from .numerics import io_round as _io_round


def _io(a, io: str) -> np.ndarray:
    if io == "f64":
        return np.asarray(a, dtype=np.float64)
    return _io_round(a, io)


def logsigmoid(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore", divide="ignore"):
        return np.log(1.0 / (1.0 + np.exp(-x)))


def multistep(c, n, m, q, k, v, i, f, eps: float, io: str = "bf16", qk_scale: float | None = None,
              literal_gate: bool = False):
    """c [NH, DQ, DV], n [NH, DQ], m [NH]; q, k [T, NH, DQ]; v [T, NH, DV]; i, f [T, NH] (float values).

    Returns (h [T, NH, DV] float64 values of the io dtype, (c_T, n_T, m_T) float64)."""
    C = np.array(c, dtype=np.float64)
    N = np.array(n, dtype=np.float64)
    M = np.array(m, dtype=np.float64).reshape(-1)
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    i = np.asarray(i, dtype=np.float64).reshape(q.shape[0], -1)
    f = np.asarray(f, dtype=np.float64).reshape(q.shape[0], -1)
    T, NH, DQ = q.shape
    DV = v.shape[-1]
    scale = DQ ** -0.5 if qk_scale is None else qk_scale
    h = np.zeros((T, NH, DV), dtype=np.float64)
    with np.errstate(over="ignore", under="ignore"):
        for t in range(T):
            fl = f[t] if literal_gate else logsigmoid(f[t])
            m_new = np.maximum(fl + M, i[t])
            fa = _io(np.exp(fl + M - m_new), io)
            ia = _io(np.exp(i[t] - m_new), io)
            mv = _io(np.exp(-m_new), io)
            C = fa[:, None, None] * C + ia[:, None, None] * (k[t][:, :, None] * v[t][:, None, :])
            N = fa[:, None] * N + ia[:, None] * k[t]
            qs = q[t] * scale
            hnum = np.einsum("hd,hdv->hv", qs, _io(C, io))
            qn = np.einsum("hd,hd->h", qs, _io(N, io))
            h[t] = _io(hnum / (np.maximum(np.abs(qn), mv) + eps)[:, None], io)
            M = m_new
    return h, (C, N, M)


def unstabilised(c, n, m, q, k, v, i, f, qk_scale: float | None = None) -> np.ndarray:
    """h [T, NH, DV] of the unstabilised recurrence in float64 (no roundings, eps = 0)."""
    M0 = np.asarray(m, dtype=np.float64).reshape(-1)
    C = np.array(c, dtype=np.float64) * np.exp(M0)[:, None, None]
    N = np.array(n, dtype=np.float64) * np.exp(M0)[:, None]
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    i = np.asarray(i, dtype=np.float64).reshape(q.shape[0], -1)
    f = np.asarray(f, dtype=np.float64).reshape(q.shape[0], -1)
    T, NH, DQ = q.shape
    scale = DQ ** -0.5 if qk_scale is None else qk_scale
    h = np.zeros((T, NH, v.shape[-1]), dtype=np.float64)
    for t in range(T):
        sf = 1.0 / (1.0 + np.exp(-f[t]))
        ei = np.exp(i[t])
        C = sf[:, None, None] * C + ei[:, None, None] * (k[t][:, :, None] * v[t][:, None, :])
        N = sf[:, None] * N + ei[:, None] * k[t]
        qs = q[t] * scale
        h[t] = np.einsum("hd,hdv->hv", qs, C) / np.maximum(np.abs(np.einsum("hd,hd->h", qs, N)), 1.0)[:, None]
    return h
