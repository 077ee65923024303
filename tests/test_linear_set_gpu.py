"""GPU parity of the persistent decode-step set kernel (optim/linear_set.py, csrc/linear_set.hip).

Every stage records the input vector it used (x_used), so each stage is checked on its own against the oracle:
  - its outputs against oracle.skinny on that input (componentwise < 4e-3 and normwise < 1e-2, the skinny gates);
  - its input against oracle.linear_set.unit_rms of the output it depends on (equal up to one bf16 step where the
    float32 and float64 mean squares round differently), which also shows the stage waited for that output: a
    stage that read its source early would have used a stale vector.
Full-size checks use the reference's own fp32 formulation (x.float() @ W.float().T) on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd import decode_set as D
from byteprof_amd.optim.linear_set import LinearSet, Stage
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import linear_set as OL
from oracle import numerics as ON
from oracle import skinny as OS
from tests.helpers import TOL_COMPONENTWISE, TOL_NORMWISE

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _np(t):
    return t.float().cpu().numpy()


def _bf16_step_close(a, b) -> bool:
    """a, b bf16 values (float arrays): equal, or one bf16 step apart."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    ua = a.view(np.uint32).astype(np.int64) >> 16
    ub = b.view(np.uint32).astype(np.int64) >> 16
    same_sign = np.sign(a) == np.sign(b)
    return bool(np.all((a == b) | (same_sign & (np.abs(ua - ub) <= 1))))


def _weights(kind, n, k, g, scale_dtype=torch.bfloat16):
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    if kind == "bf16":
        return w, None, _np(w)
    q, s = quantize_rowwise_int8(w, scale_dtype)
    return q, s, (q.cpu().numpy(), s.float().cpu().numpy())


def _small_chain(kind, seed=0, scale_dtype=torch.bfloat16):
    """Ragged stages: N below and above the grid's compute-wave count, several weight segments, K = 1024..8192,
    dependent stages reading slices of earlier outputs, renormalised and not."""
    g = _gen(seed)
    specs = [  # (segment rows, K, source: None | (stage, start), renorm)
        ([300, 1000, 77], 1024, None, False),
        ([5000], 1024, (0, 0), True),          # reads stage 0's first 1024 outputs
        ([64, 2111], 4096, (1, 904), True),    # reads stage 1 from an offset
        ([1], 2048, (2, 0), False),            # a single row: most waves have none
        ([3000, 3000, 10, 4096], 2048, (2, 96), True),
        ([2048], 8192, None, False),           # an independent stage after dependent ones
    ]
    if kind == "int8":
        specs = [(r, max(k, 1024), s, n) for r, k, s, n in specs]
    stages, ostages = [], []
    for rows, k, src, renorm in specs:
        ws, ss, ows = [], [], []
        for n in rows:
            w, s, ow = _weights(kind, n, k, g, scale_dtype)
            ws.append(w)
            ss.append(s)
            ows.append(ow)
        out = torch.empty(sum(rows), dtype=torch.bfloat16, device=DEV)
        xu = torch.empty(k, dtype=torch.bfloat16, device=DEV)
        if src is None:
            x = torch.randn(k, generator=g, device=DEV).to(torch.bfloat16)
            stages.append(Stage(ws, x, out, scales=ss if kind == "int8" else None, renorm=renorm, x_used=xu))
            ostages.append(OL.OracleStage(ows, ("ext", _np(x)), renorm, kind))
        else:
            idx, start = src
            view = stages[idx].out[start:start + k]
            stages.append(Stage(ws, view, out, scales=ss if kind == "int8" else None, wait=idx, renorm=renorm,
                                x_used=xu))
            ostages.append(OL.OracleStage(ows, ("stage", idx, start), renorm, kind))
    return stages, ostages


def _check_stages(stages, ostages):
    ys = [_np(st.out) for st in stages]
    for i, (st, ost) in enumerate(zip(stages, ostages)):
        x_used = _np(st.x_used)
        expect_x = OL.stage_input(ost, ys)  # from the GPU's own outputs of earlier stages
        assert _bf16_step_close(x_used, expect_x), f"stage {i}: input differs from its source"
        y = ys[i]
        y_ref = OL.stage_output(ost, x_used)
        w_all = np.concatenate([w if ost.kind == "bf16" else OS.dequantize("int8", *w) for w in ost.weights])
        comp = ON.componentwise_error(y[None, :], x_used[None, :], w_all)
        norm = ON.normwise_error(y, OS.matmul(x_used[None, :], w_all)[0])
        assert comp < TOL_COMPONENTWISE, (i, comp)
        assert norm < TOL_NORMWISE, (i, norm)
        # outputs are bf16 of an fp32 sum: at most one bf16 step from the float64 oracle's rounding
        assert np.mean(y == y_ref) > 0.97, i


@pytest.mark.parametrize("kind,scale_dtype", [("bf16", None), ("int8", torch.bfloat16), ("int8", torch.float16)])
def test_small_chain_matches_the_oracle_stage_by_stage(kind, scale_dtype):
    stages, ostages = _small_chain(kind, seed=3, scale_dtype=scale_dtype or torch.bfloat16)
    ls = LinearSet(stages)
    ls.run()
    torch.cuda.synchronize()
    assert not ls.timed_out()
    _check_stages(stages, ostages)


def test_int8_rows_of_two_chunks_at_extreme_input_scales():
    """int8 rows of K = 2048 go through the fp16 form of the weights against x * 2^e (e per lane from its largest
    |x|): inputs from 1e-30 to 3e4, a single large outlier among tiny values, and an all-zero input, each checked
    against the oracle (the zero input must give exact zeros)."""
    g = _gen(11)
    k = 2048
    base = torch.randn(k, generator=g, device=DEV)
    outlier = torch.full((k,), 1e-3, device=DEV)
    outlier[5] = 3.0e4
    inputs = [base * 1e4, base * 1e-4, base * 1e-30, outlier, torch.zeros(k, device=DEV)]
    stages, ostages = [], []
    for x in inputs:
        w, sc, ow = _weights("int8", 777, k, g, torch.float16)
        xb = x.to(torch.bfloat16)
        out = torch.empty(777, dtype=torch.bfloat16, device=DEV)
        stages.append(Stage([w], xb, out, scales=[sc], x_used=torch.empty(k, dtype=torch.bfloat16, device=DEV)))
        ostages.append(OL.OracleStage([ow], ("ext", _np(xb)), False, "int8"))
    ls = LinearSet(stages)
    ls.run()
    torch.cuda.synchronize()
    assert not ls.timed_out()
    _check_stages(stages, ostages)
    assert torch.count_nonzero(stages[-1].out) == 0


def test_repeated_launches_are_deterministic_and_need_no_reset():
    stages, ostages = _small_chain("bf16", seed=4)
    ls = LinearSet(stages)
    outs = []
    for _ in range(4):  # the counters keep growing; each launch waits for its own generation
        for st in stages:
            st.out.fill_(7.0)
        ls.run()
        torch.cuda.synchronize()
        outs.append([st.out.clone() for st in stages])
    assert not ls.timed_out()
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)
    _check_stages(stages, ostages)


def test_graph_replays_match_eager():
    stages, _ = _small_chain("bf16", seed=5)
    ls = LinearSet(stages)
    ls.run()
    torch.cuda.synchronize()
    eager = [st.out.clone() for st in stages]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ls.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ls.run()
    for _ in range(3):
        for st in stages:
            st.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, st in zip(eager, stages):
            assert torch.equal(a, st.out)
    assert not ls.timed_out()


def test_input_change_between_launches_is_seen():
    stages, ostages = _small_chain("bf16", seed=6)
    ls = LinearSet(stages)
    ls.run()
    stages[0].src.copy_(torch.randn(stages[0].k, generator=_gen(60), device=DEV).to(torch.bfloat16))
    ostages[0].src = ("ext", _np(stages[0].src))
    ls.run()
    torch.cuda.synchronize()
    _check_stages(stages, ostages)


def test_fresh_inputs_on_every_launch_reach_every_stage():
    """A new external input before each launch: every dependent stage must see this launch's rows (a stage that
    read a row before its producer published it would see the previous launch's value, which differs)."""
    stages, ostages = _small_chain("bf16", seed=7)
    ls = LinearSet(stages)
    for it in range(6):
        x = torch.randn(stages[0].k, generator=_gen(700 + it), device=DEV).to(torch.bfloat16)
        stages[0].src.copy_(x)
        ostages[0].src = ("ext", _np(x))
        ls.run()
        torch.cuda.synchronize()
        _check_stages(stages, ostages)
    assert not ls.timed_out()


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("dependent", [True, False])
def test_full_decode_step_set(kind, dependent):
    """The OLMo-2-1B-shaped set (16 layers x q|k|v, o, gate|up, down + the 100352-row head) in one launch."""
    ch = D.build_chain(kind, DEV, seed=11, dependent=dependent, record_inputs=True)
    ch.lset.run()
    if dependent:  # a second launch with a new first input: every stage must see this launch's values
        ch.stages[0].src.copy_(torch.randn(ch.stages[0].k, generator=_gen(12), device=DEV).to(torch.bfloat16))
        ch.lset.run()
    torch.cuda.synchronize()
    assert not ch.lset.timed_out()
    assert len(ch.stages) == 16 * 4 + 1
    ys_host = [_np(st.out) for st in ch.stages]
    for i, st in enumerate(ch.stages):
        x = st.x_used.float()
        if st.wait >= 0:
            base = ch.stages[st.wait].out
            start = (st.src.data_ptr() - base.data_ptr()) // 2
            src = ys_host[st.wait][start:start + st.k]
            assert _bf16_step_close(_np(st.x_used), OL.unit_rms(src)), i
        elif st.renorm:
            assert _bf16_step_close(_np(st.x_used), OL.unit_rms(_np(st.src))), i
        else:
            assert torch.equal(st.x_used, st.src)
        if kind == "bf16":
            w = torch.cat([w.float() for w in st.weights])
        else:
            w = torch.cat([q.float() * s.float()[:, None] for q, s in zip(st.weights, st.scales)])
        ref = x @ w.T  # the reference's fp32 formulation (tests/test_skinny.py:38)
        y = st.out.float()
        norm = float((y - ref).abs().max() / ref.abs().max())
        comp = float(((y - ref).abs() / (x.abs() @ w.abs().T).clamp_min(1e-30)).max())
        assert norm < TOL_NORMWISE, (i, norm)
        assert comp < TOL_COMPONENTWISE, (i, comp)
        if i == len(ch.stages) - 1:  # greedy argmax over the LM head
            ref_bf = ref.to(torch.bfloat16).float()
            top2 = torch.topk(ref, 2).values
            if float(top2[0] - top2[1]) > 2.0 ** -6 * float(top2[0].abs()):
                assert int(torch.argmax(y)) == int(torch.argmax(ref_bf))
        del w, ref
