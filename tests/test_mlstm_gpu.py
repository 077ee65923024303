"""Fused multi-step mLSTM kernel on the GPU against the CPU oracle (oracle/mlstm.py): T = 1..33 positions, one- and
multi-block head dims (64, 128, 256), fp32 and bf16 inputs, every value block, the 4-head 256-wide configuration,
the read-only start state, the saved start n/m, graph capture. Mirrors byteprof tests/test_fused_kernels_gpu.py
(the reference compares against mlstm_kernels' step kernel, which is not available here: the oracle restates the
arithmetic of byteprof/optim/mlstm_multistep.py and is itself pinned by tests/test_oracle.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd.optim import draft_fused as F
from oracle import mlstm as OM
from oracle import numerics as ON

pytestmark = pytest.mark.gpu

IO = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def rand_inputs(t, nh, dq, dv, dtype, seed=0, gate_dtype=None, f_mean=0.0, gate_scale=2.0):
    """Seeded inputs; the reference test's distributions (tests/test_fused_kernels_gpu.py:15-20) by default."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    gate_dtype = gate_dtype or dtype

    def r(*shape, dt=dtype):
        return torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32).to(dt)

    q, k, v = r(t, nh, dq), r(t, nh, dq), r(t, nh, dv)
    i = (r(t, nh, 1, dt=torch.float32) * gate_scale).to(gate_dtype)
    f = (r(t, nh, 1, dt=torch.float32) * gate_scale + f_mean).to(gate_dtype)
    state = (r(1, nh, dq, dv, dt=torch.float32) * 0.1, r(1, nh, dq, dt=torch.float32) * 0.1,
             r(1, nh, 1, dt=torch.float32))
    return q, k, v, i, f, state


def oracle(state, q, k, v, i, f, eps, io):
    c, n, m = (x.cpu().numpy() for x in state)
    h, st = OM.multistep(c[0], n[0], m[0].reshape(-1), q.float().cpu().numpy(), k.float().cpu().numpy(),
                         v.float().cpu().numpy(), i.float().cpu().numpy().reshape(q.shape[0], -1),
                         f.float().cpu().numpy().reshape(q.shape[0], -1), eps=eps, io=io)
    return h, st


def run(state, q, k, v, i, f, eps=1e-6, bv=None, hrows=None):
    t, nh, dq = q.shape
    dv = v.shape[-1]
    hbuf = torch.zeros(hrows or t, nh, dv, dtype=q.dtype, device="cuda")
    ns, ms = torch.zeros(nh, dq, device="cuda"), torch.zeros(nh, device="cuda")
    F.multistep_fw(state, q, k, v, i, f, hbuf, ns, ms, eps=eps, bv=bv)
    return hbuf, ns, ms


@pytest.mark.parametrize("dq", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_outputs_match_the_oracle_for_every_t(dtype, dq):
    nh, dv = 16, 128
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    worst = 0.0
    for t in (1, 2, 5, 9, 17, 33):
        print(f"\n[mlstm] dtype={dtype} dq={dq} t={t}", flush=True)
        q, k, v, i, f, state = rand_inputs(t, nh, dq, dv, dtype, seed=t)
        start = tuple(x.clone() for x in state)
        hbuf, ns, ms = run(state, q, k, v, i, f, hrows=40)
        assert all(torch.equal(a, b) for a, b in zip(state, start))  # the pass never writes the state
        assert torch.equal(ns, state[1][0]) and torch.equal(ms, state[2].reshape(-1))
        assert (hbuf[t:] == 0).all()  # rows past T untouched
        h_ref, _ = oracle(state, q, k, v, i, f, 1e-6, IO[dtype])
        err = ON.normwise_error(hbuf[:t].float().cpu().numpy(), h_ref)
        worst = max(worst, err)
        assert err < tol, (t, err)
    print("worst normwise error", dtype, dq, worst)


@pytest.mark.parametrize("bv", [4, 8, 16])
def test_every_value_block_gives_the_same_outputs(bv):
    q, k, v, i, f, state = rand_inputs(7, 4, 128, 64, torch.bfloat16, seed=3)
    h_ref, _ = oracle(state, q, k, v, i, f, 1e-6, "bf16")
    hbuf, _, _ = run(state, q, k, v, i, f, bv=bv)
    assert ON.normwise_error(hbuf.float().cpu().numpy(), h_ref) < 1e-2


def test_the_four_head_256_wide_configuration():
    """NH = 4, DQ = DV = 256, T = 16; bf16 q/k/v, fp32 gate pre-activations i ~ N(0,1), f ~ N(3,1); fp32 state
    drawn N(0, 0.1^2) (m ~ N(0, 1)). Normwise error <= 1e-2 against the oracle, and the fp32 run against the
    unstabilised closed form."""
    q, k, v, i, f, state = rand_inputs(16, 4, 256, 256, torch.bfloat16, seed=2024, gate_dtype=torch.float32,
                                       f_mean=3.0, gate_scale=1.0)
    h_ref, _ = oracle(state, q, k, v, i, f, 1e-6, "bf16")
    hbuf, _, _ = run(state, q, k, v, i, f)
    assert ON.normwise_error(hbuf.float().cpu().numpy(), h_ref) < 1e-2
    q32, k32, v32 = (x.float() for x in (q, k, v))
    h32, _, _ = run(state, q32, k32, v32, i, f, eps=0.0)
    c, n, m = (x.cpu().numpy() for x in state)
    closed = OM.unstabilised(c[0], n[0], m.reshape(-1), q32.cpu().numpy(), k32.cpu().numpy(), v32.cpu().numpy(),
                             i.cpu().numpy().reshape(16, -1), f.cpu().numpy().reshape(16, -1))
    assert ON.normwise_error(h32.cpu().numpy(), closed) < 1e-5


def test_strided_positions():
    """q, k, v, i, f, h as views with a position stride larger than the row (as slices of bigger buffers)."""
    q, k, v, i, f, state = rand_inputs(6, 2, 64, 32, torch.bfloat16, seed=9)
    big = lambda x: torch.cat([x, torch.zeros_like(x)], dim=1)[:, :x.shape[1]]  # noqa: E731
    qs, ks, vs = big(q), big(k), big(v)
    i2 = torch.cat([i, i], dim=1)[:, :2]
    f2 = torch.cat([f, f], dim=1)[:, :2]
    assert qs.stride(0) == 2 * 2 * 64 and not qs.is_contiguous()
    hb = torch.zeros(6, 4, 32, dtype=torch.bfloat16, device="cuda")
    h = hb[:, :2]
    ns, ms = torch.zeros(2, 64, device="cuda"), torch.zeros(2, device="cuda")
    F.multistep_fw(state, qs, ks, vs, i2, f2, h, ns, ms, eps=1e-6)
    h_ref, _ = oracle(state, q, k, v, i, f, 1e-6, "bf16")
    assert ON.normwise_error(h.float().cpu().numpy(), h_ref) < 1e-2
    assert (hb[:, 2:] == 0).all()


def test_inside_a_hip_graph_with_changing_inputs():
    q, k, v, i, f, state = rand_inputs(9, 4, 128, 64, torch.bfloat16, seed=4)
    hbuf = torch.zeros(9, 4, 64, dtype=torch.bfloat16, device="cuda")
    ns, ms = torch.zeros(4, 128, device="cuda"), torch.zeros(4, device="cuda")
    F.multistep_fw(state, q, k, v, i, f, hbuf, ns, ms, eps=1e-6)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        F.multistep_fw(state, q, k, v, i, f, hbuf, ns, ms, eps=1e-6)
    for seed in range(3):
        q2, k2, v2, i2, f2, _ = rand_inputs(9, 4, 128, 64, torch.bfloat16, seed=50 + seed)
        for dst, src in ((q, q2), (k, k2), (v, v2), (i, i2), (f, f2)):
            dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        h_ref, _ = oracle(state, q, k, v, i, f, 1e-6, "bf16")
        assert ON.normwise_error(hbuf.float().cpu().numpy(), h_ref) < 1e-2
        eager = torch.zeros_like(hbuf)
        F.multistep_fw(state, q, k, v, i, f, eager, ns, ms, eps=1e-6)
        assert torch.equal(eager, hbuf)


def test_zero_positions_only_saves_the_start_state():
    _, _, _, _, _, state = rand_inputs(1, 2, 64, 16, torch.float32, seed=1)
    q = torch.zeros(0, 2, 64, device="cuda")
    v = torch.zeros(0, 2, 16, device="cuda")
    g = torch.zeros(0, 2, 1, device="cuda")
    h = torch.zeros(1, 2, 16, device="cuda")
    ns, ms = torch.zeros(2, 64, device="cuda"), torch.zeros(2, device="cuda")
    F.multistep_fw(state, q, q, v, g, g, h, ns, ms, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(ns, state[1][0]) and torch.equal(ms, state[2].reshape(-1)) and (h == 0).all()
    assert np.isfinite(ns.cpu().numpy()).all()


def _step(state, q, k, v, i, f, eps=1e-6, bv=None):
    from byteprof_amd.optim import draft_core as DC

    nh, dv = q.shape[1], v.shape[-1]
    new = tuple(torch.full_like(x, float("nan")) for x in state)
    h = torch.zeros(1, nh, dv, dtype=q.dtype, device="cuda")
    DC.mlstm_step_into(state, new, q, k, v, i, f, h, eps, bv=bv)
    return h, new


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("nh,dq,dv", [(4, 256, 256), (16, 128, 128), (2, 512, 64)])
def test_step_matches_the_oracle(dtype, nh, dq, dv):
    """mlstm_step_into (bp_mlstm_step): h and the new state of one position against the oracle at T = 1; the
    previous state is left as it was."""
    print(f"\n[mlstm step] dtype={dtype} nh={nh} dq={dq} dv={dv}", flush=True)
    q, k, v, i, f, state = rand_inputs(1, nh, dq, dv, dtype, seed=11, f_mean=3.0)
    start = tuple(x.clone() for x in state)
    h, new = _step(state, q, k, v, i, f)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(state, start))
    h_ref, (c_ref, n_ref, m_ref) = oracle(state, q, k, v, i, f, 1e-6, IO[dtype])
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert ON.normwise_error(h.float().cpu().numpy(), h_ref) < tol
    assert ON.normwise_error(new[0].cpu().numpy().reshape(c_ref.shape), c_ref) < 1e-5
    assert ON.normwise_error(new[1].cpu().numpy().reshape(n_ref.shape), n_ref) < 1e-5
    assert np.allclose(new[2].cpu().numpy().reshape(-1), m_ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bv", [4, 8, 16])
def test_step_equals_multistep_then_lazy_commit(dtype, bv):
    """One step equals the fused multistep over one position (h) followed by the lazy commit of L = 0 (the state),
    bit for bit."""
    q, k, v, i, f, state = rand_inputs(1, 4, 256, 256, dtype, seed=12)
    h, new = _step(state, q, k, v, i, f, bv=bv)
    cur = tuple(x.clone() for x in state)
    h1 = torch.zeros_like(h)
    ns, ms = torch.zeros(4, 256, device="cuda"), torch.zeros(4, device="cuda")
    F.multistep_fw(cur, q, k, v, i, f, h1, ns, ms, eps=1e-6, bv=bv)
    F.lazy_commit(cur, k, v, i, f, torch.tensor(0, device="cuda"), ns, ms, bv=bv)
    torch.cuda.synchronize()
    assert torch.equal(h, h1)
    for a, b in zip(new, cur):
        assert torch.equal(a.reshape(-1), b.reshape(-1))


def test_step_refuses_overlapping_state():
    from byteprof_amd.optim import draft_core as DC

    q, k, v, i, f, state = rand_inputs(1, 2, 64, 16, torch.bfloat16, seed=13)
    h = torch.zeros(1, 2, 16, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        DC.mlstm_step_into(state, state, q, k, v, i, f, h, 1e-6)
