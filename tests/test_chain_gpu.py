"""GPU parity of the one-launch linear set (optim/linear_chain.py, csrc/skinny_chain.hip).

  - independent stages (external inputs): every output bitwise equal to skinny_mm at M = 1 with the same plan
    (weight blocks, waves, split 1), and within the skinny gates of the oracle;
  - dependent stages: each stage's outputs against the oracle on the input it should have waited for (the unit-RMS
    renormalisation, oracle.linear_set.unit_rms, of the slice of its producer's output), componentwise < 4e-3 and
    normwise < 1e-2 -- a stage that read its source early would have used a stale vector;
  - repeated launches need no reset and are deterministic; graph replays equal eager launches; a new external
    input reaches every dependent stage; no wait ever gives up;
  - the full decode-step set (bf16, int8), dependent and independent.
Full-size checks use the reference's own fp32 formulation (x.float() @ W.float().T) on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd import decode_set as D
from byteprof_amd.optim import skinny as S
from byteprof_amd.optim.linear_chain import ChainStage, LinearChain
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import linear_set as OL
from oracle import skinny as OS
from tests.helpers import check_against_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _weights(kind, n, k, g, scale_dtype=torch.bfloat16):
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    return w if kind == "bf16" else quantize_rowwise_int8(w, scale_dtype)


def _oracle_w(w) -> np.ndarray:
    if isinstance(w, tuple):
        return OS.dequantize("int8", w[0].cpu().numpy(), w[1].float().cpu().numpy())
    return w.float().cpu().numpy()


def _small_stages(kind, seed=0, scale_dtype=torch.bfloat16):
    """Ragged stages: row counts below and above a workgroup, several weights per stage, K = 1024..8192, dependent
    stages reading slices of earlier outputs, renormalised and not, an independent stage after dependent ones."""
    g = _gen(seed)
    specs = [  # (rows per weight, K, source: None | (stage, start), renorm)
        ([300, 1000, 77], 1024, None, False),
        ([5000], 1024, (0, 0), True),
        ([64, 2111], 4096, (1, 904), True),
        ([1], 2048, (2, 0), False),
        ([3000, 3000, 10, 4096], 2048, (2, 96), True),
        ([2048], 8192, None, False),
        ([700], 2048, (4, 5000), True),  # the last stage reads the one before the independent stage
    ]
    stages = []
    for rows, k, src, renorm in specs:
        ws = [_weights(kind, n, k, g, scale_dtype) for n in rows]
        out = torch.empty(sum(rows), dtype=torch.bfloat16, device=DEV)
        x = torch.randn(k, generator=g, device=DEV).to(torch.bfloat16) if src is None else src
        stages.append(ChainStage(ws, x, out, renorm))
    return stages


def _check_stage(stages, i):
    """Stage i's outputs against the oracle on the input it should have used (its external x, or the oracle's
    renormalisation of its producer's actual output)."""
    st = stages[i]
    k = int((st.weights[0][0] if isinstance(st.weights[0], tuple) else st.weights[0]).shape[1])
    if isinstance(st.src, tuple):
        dep, start = st.src
        src = stages[dep].out[start:start + k].float().cpu().numpy()
    else:
        src = st.src.float().cpu().numpy()
    x = OL.unit_rms(src) if st.renorm else src
    w = np.concatenate([_oracle_w(w) for w in st.weights])
    xt = torch.tensor(x[None], dtype=torch.float32).to(torch.bfloat16).to(DEV)
    return check_against_oracle(st.out[None], xt, w)


@pytest.mark.parametrize("kind,scale_dtype", [("bf16", None), ("int8", torch.bfloat16), ("int8", torch.float16)])
@pytest.mark.parametrize("plan", [(0, 8), (2, 8), (1, 4), (4, 2)])
def test_small_chain_matches_the_oracle_stage_by_stage(kind, scale_dtype, plan):
    print(f"\n[chain] {kind} {scale_dtype} rb={plan[0]} waves={plan[1]}", flush=True)
    stages = _small_stages(kind, seed=1, scale_dtype=scale_dtype or torch.bfloat16)
    ch = LinearChain(stages, rb=plan[0], waves=plan[1])
    assert ch.dependent
    for rep in range(3):
        ch.run()
    torch.cuda.synchronize()
    assert not ch.timed_out()
    for i in range(len(stages)):
        _check_stage(stages, i)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("plan", [(0, 8), (2, 8), (1, 4), (4, 2), (0, 2)])
def test_independent_stages_equal_skinny_mm(kind, plan):
    """Without dependencies every output is the skinny_mm output with the same waves (split 1), bit for bit,
    whatever the rows per workgroup."""
    g = _gen(3)
    shapes = [(300, 1024), (5000, 2048), (1, 4096), (2111, 8192), (64, 2048), (100352 // 7, 2048)]
    stages, refs = [], []
    for n, k in shapes:
        w = _weights(kind, n, k, g, torch.float16)
        x = torch.randn(k, generator=g, device=DEV).to(torch.bfloat16)
        stages.append(ChainStage([w], x, torch.empty(n, dtype=torch.bfloat16, device=DEV)))
        args = w if isinstance(w, tuple) else (w,)
        refs.append((x, args))
    ch = LinearChain(stages, rb=plan[0], waves=plan[1])
    assert not ch.dependent
    ch.run()
    for st, (x, args) in zip(stages, refs):
        want = S.skinny_mm(x[None], *args, cfg=(8 * max(plan[0], 1), plan[1], 1))[0]
        assert torch.equal(st.out, want), st.out.numel()
        check_against_oracle(st.out[None], x[None], _oracle_w(st.weights[0]))


def test_repeated_launches_need_no_reset_and_are_deterministic():
    stages = _small_stages("bf16", seed=2)
    ch = LinearChain(stages)
    ch.run()
    first = [st.out.clone() for st in stages]
    for _ in range(5):
        ch.run()
    torch.cuda.synchronize()
    assert not ch.timed_out()
    for st, f in zip(stages, first):
        assert torch.equal(st.out, f)


def test_graph_replays_match_eager_and_new_inputs_reach_every_stage():
    """Captured once, replayed with new external inputs and eager work in between: every replay equals an eager
    launch on the same inputs, and every dependent stage changes with the input."""
    stages = _small_stages("int8", seed=4, scale_dtype=torch.float16)
    ch = LinearChain(stages)
    ch.run()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ch.run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ch.run()
    prev = None
    for seed in range(4):
        stages[0].src.copy_(torch.randn(stages[0].src.numel(), generator=_gen(100 + seed), device=DEV))
        _ = torch.randn(1000, device=DEV).sum()
        g.replay()
        torch.cuda.synchronize()
        got = [st.out.clone() for st in stages]
        ch.run()
        torch.cuda.synchronize()
        for i, st in enumerate(stages):
            assert torch.equal(got[i], st.out), (seed, i)
        if prev is not None:
            for i in (0, 1, 2, 3, 4, 6):  # the stages that depend on stage 0's input
                assert not torch.equal(prev[i], got[i]), (seed, i)
        prev = got
    assert not ch.timed_out()


def _check_decode_stages(chain):
    """Every stage's outputs against the fp32 product of its input as the chain defines it (the renormalised slice
    of its producer's actual output, or its own vector)."""
    for i, st in enumerate(chain.stages):
        k = int((st.weights[0][0] if isinstance(st.weights[0], tuple) else st.weights[0]).shape[1])
        if isinstance(st.src, tuple):
            dep, start = st.src
            src = chain.stages[dep].out[start:start + k]
        else:
            src = st.src
        x = D.unit_rms(src[None]) if st.renorm else src[None]
        w32 = torch.cat([(w[0].float() * w[1].float()[:, None]) if isinstance(w, tuple) else w.float()
                         for w in st.weights])
        ref = x.float() @ w32.T
        den = (x.float().abs() @ w32.abs().T).clamp(min=1e-30)
        comp = float(((st.out[None].float() - ref).abs() / den).max())
        norm = float((st.out[None].float() - ref).abs().max() / ref.abs().max())
        assert comp < 4e-3 and norm < 1e-2, (i, comp, norm)
        del w32


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("dependent", [True, False])
def test_full_decode_step_set(kind, dependent):
    print(f"\n[chain] decode-step set {kind} dependent={dependent}", flush=True)
    weights = D.make_weights(kind, DEV, seed=0)
    chain = D.build_chain(kind, DEV, weights=weights, dependent=dependent)
    for _ in range(2):
        chain.lset.run()
    torch.cuda.synchronize()
    assert not chain.lset.timed_out()
    _check_decode_stages(chain)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_plain_stage_launches_of_the_set(kind):
    """The set as the 65 plain stage launches that bench.py times (decode_set.build_stages: one skinny launch per
    stage over its adjacent weight rows, each on its own unit-RMS input), replayed from a HIP graph: every stage's
    output against the fp32 product of its input and weights, and each replay equal to the eager pass."""
    print(f"\n[set] 65 plain stage launches {kind}", flush=True)
    weights = D.make_weights(kind, DEV, seed=0)
    ops = D.build_stages(weights, 1, DEV, seed=0)
    assert len(ops) == 65
    for op in ops:
        op()
    torch.cuda.synchronize()
    for i, op in enumerate(ops):
        w = op.args
        w32 = (w[0].float() * w[1].float()[:, None]) if len(w) > 1 else w[0].float()
        ref = op.x.float() @ w32.T
        den = (op.x.float().abs() @ w32.abs().T).clamp(min=1e-30)
        comp = float(((op.y.float() - ref).abs() / den).max())
        norm = float((op.y.float() - ref).abs().max() / ref.abs().max())
        assert comp < 4e-3 and norm < 1e-2, (i, op.name, comp, norm)
        del w32
    eager = [op.y.clone() for op in ops]
    g = D.capture(ops)
    for _ in range(3):
        for op in ops:
            op.y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, op.y) for a, op in zip(eager, ops))


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_stage_graph_of_skinny_launches(kind):
    """The dependent set as 65 stream-ordered skinny launches (one per stage over its adjacent weight rows, the
    renormalisation inside the launch), eager and replayed from a HIP graph: every stage within the gates of its
    input; replays equal the eager pass."""
    print(f"\n[chain] stage graph of skinny launches {kind}", flush=True)
    weights = D.make_weights(kind, DEV, seed=0)
    chain = D.build_chain(kind, DEV, weights=weights, dependent=True)
    calls = D.stage_graph_calls(chain)
    assert len(calls) == 65
    for c in calls:
        c()
    torch.cuda.synchronize()
    _check_decode_stages(chain)
    eager = [st.out.clone() for st in chain.stages]
    g = D.capture(calls)
    for _ in range(3):
        for st in chain.stages:
            st.out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, st.out) for a, st in zip(eager, chain.stages))
