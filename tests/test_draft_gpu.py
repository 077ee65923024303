"""Drafting-round kernels on the GPU against the CPU oracle: lazy commit of the accepted prefix (dynamic length in
a captured graph, state updated in place), the accepted-length kernel, and the commit of a history slot. Mirrors
byteprof tests/test_fused_kernels_gpu.py:85-126."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd.optim import draft_core as DC
from byteprof_amd.optim import draft_fused as F
from oracle import draft as OD
from oracle import numerics as ON
from tests.test_mlstm_gpu import IO, rand_inputs

pytestmark = pytest.mark.gpu


def _oracle_state(start, k, v, i, f, length, io):
    c, n, m = (x.cpu().numpy() for x in start)
    return OD.committed_state(c[0], n[0], m[0].reshape(-1), k.float().cpu().numpy(), v.float().cpu().numpy(),
                              i.float().cpu().numpy().reshape(k.shape[0], -1),
                              f.float().cpu().numpy().reshape(k.shape[0], -1), length, io)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("nh,dq,dv", [(16, 64, 128), (4, 256, 256), (2, 512, 64)])
def test_lazy_commit_in_a_graph_with_a_dynamic_length(dtype, nh, dq, dv):
    t = 7
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    q, k, v, i, f, state = rand_inputs(t, nh, dq, dv, dtype, seed=3)
    start = tuple(x.clone() for x in state)
    cur = tuple(x.clone() for x in state)
    hbuf = torch.zeros(8, nh, dv, dtype=dtype, device="cuda")
    ns, ms = torch.zeros(nh, dq, device="cuda"), torch.zeros(nh, device="cuda")
    length = torch.zeros((), dtype=torch.long, device="cuda")
    F.multistep_fw(cur, q, k, v, i, f, hbuf, ns, ms, eps=1e-6)
    F.lazy_commit(cur, k, v, i, f, length, ns, ms)
    torch.cuda.synchronize()
    for a, b in zip(cur, start):
        a.copy_(b)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        F.multistep_fw(cur, q, k, v, i, f, hbuf, ns, ms, eps=1e-6)
        F.lazy_commit(cur, k, v, i, f, length, ns, ms)
    for length_v in (0, 3, t - 1, 1, t + 5):
        print(f"\n[lazy_commit] dtype={dtype} nh={nh} dq={dq} dv={dv} L={length_v}", flush=True)
        for a, b in zip(cur, start):
            a.copy_(b)
        length.fill_(length_v)
        g.replay()
        torch.cuda.synchronize()
        want = _oracle_state(start, k, v, i, f, length_v, IO[dtype])
        for got, ref in zip(cur, want):
            err = ON.normwise_error(got.cpu().numpy().reshape(ref.shape), ref)
            assert err < tol, (length_v, err)


def test_lazy_commit_with_no_accepted_position_keeps_the_start_state():
    q, k, v, i, f, state = rand_inputs(4, 4, 128, 64, torch.bfloat16, seed=1)
    cur = tuple(x.clone() for x in state)
    ns, ms = state[1][0].clone(), state[2].reshape(-1).clone()
    cur[1].zero_()
    cur[2].zero_()
    F.lazy_commit(cur, k, v, i, f, torch.tensor(-1, device="cuda"), ns, ms)
    assert torch.equal(cur[0], state[0]) and torch.equal(cur[1], state[1]) and torch.equal(cur[2], state[2])


def test_accept_known_answers_and_random_cases():
    ids = torch.tensor([10, 5, 6, 7, 8, 9], device="cuda")
    for tokl, want in (([5, 6, 99, 8, 9, 3], 2), ([5, 6, 7, 8, 9 + 260, 3], 4), ([1, 6, 7, 8, 9, 3], 0),
                       ([5, 6, 7, 8, 9, 3], 5)):
        tok = torch.tensor(tokl, device="cuda")
        out = torch.zeros(8, dtype=torch.long, device="cuda")
        F.accept(ids, tok, out, 6, 6)
        assert int(out[6]) == want == int(DC.accepted_length_t(ids, tok, 6))
        assert out[:6].tolist() == tokl
    rng = np.random.default_rng(0)
    for s in (1, 2, 33, 64, 65, 130):
        for _ in range(5):
            base = rng.integers(0, 1000, s + 1)
            tokn = base[1:].copy()
            cut = int(rng.integers(0, s + 1))
            if cut < s - 1:
                tokn[cut] = 5000  # first mismatch at cut
            ids_t = torch.from_numpy(base).cuda()
            tok_t = torch.from_numpy(tokn).cuda()
            out = torch.full((s + 3,), -7, dtype=torch.long, device="cuda")
            F.accept(ids_t, tok_t, out, s, s + 1)
            assert int(out[s + 1]) == OD.accepted_length(base, tokn, s), (s, cut)
            assert torch.equal(out[:s], tok_t[:s]) and int(out[s]) == -7


def test_commit_state_from_a_dynamic_slot_in_a_graph():
    slots, nh, dq, dv = 9, 4, 64, 32
    g0 = torch.Generator(device="cuda").manual_seed(2)
    hist = (torch.randn(slots, 1, nh, dq, dv, generator=g0, device="cuda"),
            torch.randn(slots, 1, nh, dq, generator=g0, device="cuda"),
            torch.randn(slots, 1, nh, 1, generator=g0, device="cuda"))
    cur = tuple(torch.zeros_like(h[0]) for h in hist)
    length = torch.zeros((), dtype=torch.long, device="cuda")
    DC.commit_state(hist, cur, length)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        DC.commit_state(hist, cur, length)
    for slot in (3, 0, 8, 5):
        length.fill_(slot)
        g.replay()
        torch.cuda.synchronize()
        for h, c in zip(hist, cur):
            assert torch.equal(c, h[slot]), slot
    cpu_hist = tuple(h.cpu() for h in hist)
    cpu_cur = tuple(torch.zeros_like(h[0]) for h in cpu_hist)
    DC.commit_state(cpu_hist, cpu_cur, torch.tensor(4))
    assert all(torch.equal(c, h[4]) for h, c in zip(cpu_hist, cpu_cur))
