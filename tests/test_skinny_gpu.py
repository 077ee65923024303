"""Skinny matmul kernels on the GPU against the CPU oracle: every M = 1..33 on the reference's real and odd shapes,
empty inputs and chunking, split-K and other tile configurations, bitwise row independence (the reference's test on
every shape, and across the launch buckets up to 64 rows), validation, the sentinel out-of-bounds check, unaligned
inputs, graph capture, gemv_int8 against skinny_mm. Mirrors byteprof tests/test_skinny.py:71-149."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from byteprof_amd.optim import skinny as S
from oracle import numerics as ON
from tests.helpers import check_against_oracle, make_weights, oracle_weights, randn_x

pytestmark = pytest.mark.gpu

REAL = [(2048, 2048), (8192, 2048), (2048, 8192), (1024, 2048), (2816, 2048), (2048, 2816)]
ODD = [(37, 256), (1, 128), (50, 384), (129, 640), (70, 1000), (3, 129), (16, 2047)]
KINDS = ["bf16", "int8"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", REAL + ODD)
def test_matches_the_oracle_for_every_m(kind, n, k):
    print(f"\n[skinny] kind={kind} n={n} k={k}", flush=True)
    _, args = make_weights(kind, n, k, seed=n + k)
    w_np = oracle_weights(kind, args)
    x = randn_x(33, k, seed=7)
    worst = (0.0, 0.0)
    for m in range(1, 34):
        y = S.skinny_mm(x[:m].contiguous(), *args)
        assert y.shape == (m, n) and y.dtype == torch.bfloat16
        worst = max(worst, check_against_oracle(y, x[:m], w_np))
    print("worst componentwise / normwise", worst)


@pytest.mark.parametrize("kind", KINDS)
def test_empty_input_and_many_rows(kind):
    _, args = make_weights(kind, 64, 256)
    w_np = oracle_weights(kind, args)
    assert S.skinny_mm(torch.empty(0, 256, device="cuda", dtype=torch.bfloat16), *args).shape == (0, 64)
    x = randn_x(150, 256, seed=1)  # more than MAX_M rows: chunked
    check_against_oracle(S.skinny_mm(x, *args), x, w_np)


@pytest.mark.parametrize("kind", KINDS)
def test_zero_k_writes_zeros(kind):
    w = torch.empty(8, 0, device="cuda", dtype=torch.bfloat16 if kind == "bf16" else torch.int8)
    args = (w,) if kind == "bf16" else (w, torch.ones(8, device="cuda", dtype=torch.bfloat16))
    out = torch.full((3, 8), 5.0, device="cuda", dtype=torch.bfloat16)
    S.skinny_mm(torch.empty(3, 0, device="cuda", dtype=torch.bfloat16), *args, out=out)
    assert (out == 0).all()


@pytest.mark.parametrize("kind,cfg", [("bf16", (32, 128, 4, 3, 4)), ("int8", (16, 256, 4, 3, 3)),
                                      ("bf16", (64, 64, 2, 2, 1)), ("bf16", (32, 128, 2, 2, 100)),
                                      ("bf16", (2, 16, 1)), ("int8", (4, 1, 2)), ("bf16", (8, 2, 3))])
def test_split_k_and_other_configs_match(kind, cfg):
    _, args = make_weights(kind, 192, 2048 if kind == "bf16" else 4096)
    w_np = oracle_weights(kind, args)
    for m in (1, 5, 16, 17, 33):
        x = randn_x(m, w_np.shape[1], seed=m)
        check_against_oracle(S.skinny_mm(x, *args, cfg=cfg), x, w_np)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", REAL + ODD)
def test_rows_do_not_depend_on_the_other_rows(kind, n, k):
    """byteprof tests/test_skinny.py:110-120 unchanged (rows 1, 3 and 9 of a 16-row call are the 16-row call's), on
    every shape: one kernel family and one K order serve every row count."""
    _, args = make_weights(kind, n, k)
    x = randn_x(16, k, seed=3)
    full = S.skinny_mm(x, *args)
    for m in (1, 3, 9):
        assert torch.equal(S.skinny_mm(x[:m].contiguous(), *args), full[:m]), m


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", [(2048, 2048), (2048, 8192), (129, 640), (100352, 2048)])
def test_rows_do_not_depend_on_the_launch_bucket(kind, n, k):
    """Beyond the reference's M <= 16 bucket: a row is the same in launches of 1..64 rows (activation blocks of 8,
    16, 32, 64) and in the chunked launches of more than MAX_M rows."""
    _, args = make_weights(kind, n, k)
    x = randn_x(130, k, seed=4)
    full = S.skinny_mm(x, *args)  # 64 + 64 + 2 rows
    for m in (1, 2, 5, 8, 9, 16, 17, 31, 33, 64):
        assert torch.equal(S.skinny_mm(x[:m].contiguous(), *args), full[:m]), m
    assert torch.equal(S.skinny_mm(x[64:128].contiguous(), *args), full[64:128])
    assert torch.equal(S.skinny_mm(x[128:].contiguous(), *args), full[128:])


def test_input_validation():
    w = torch.zeros(8, 128, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 64, device="cuda", dtype=torch.bfloat16), w)
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, device="cuda", dtype=torch.bfloat16)[:, ::2], w)
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, device="cuda", dtype=torch.bfloat16),
                    torch.zeros(8, 128, device="cuda", dtype=torch.int8))
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, device="cuda", dtype=torch.float32), w)
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, device="cuda", dtype=torch.bfloat16), w,
                    out=torch.empty(2, 9, device="cuda", dtype=torch.bfloat16))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [1, 3, 17])
def test_kernel_writes_only_the_output_block(kind, m):
    """Rows beyond M and columns beyond N are never written: the output sits inside a sentinel buffer."""
    n, k = 70, 384
    _, args = make_weights(kind, n, k)
    w_np = oracle_weights(kind, args)
    x = randn_x(m, k, seed=m)
    flat = torch.full((m * n + 4096,), 777.0, device="cuda", dtype=torch.bfloat16)
    out = flat[:m * n].view(m, n)
    S.skinny_mm(x, *args, out=out)
    assert torch.equal(flat[m * n:], torch.full_like(flat[m * n:], 777.0))
    assert not (out == 777.0).any()
    check_against_oracle(out, x, w_np)


@pytest.mark.parametrize("kind", KINDS)
def test_unaligned_operands_use_the_element_path(kind):
    """x starting 2 bytes into its storage (not 16-byte aligned) and a ragged K take the element-load kernel."""
    n, k = 96, 520
    _, args = make_weights(kind, n, k)
    w_np = oracle_weights(kind, args)
    buf = randn_x(1, 4 * k + 1, seed=5).reshape(-1)
    x = buf[1:1 + 4 * k].view(4, k)
    assert x.data_ptr() % 16 != 0
    check_against_oracle(S.skinny_mm(x, *args), x, w_np)


@pytest.mark.parametrize("kind", KINDS)
def test_k_past_the_buffer_range_takes_the_element_path(kind):
    """K >= 2^24: 64 activation rows would not fit one buffer resource, so every row count takes the element-load
    kernel (the same K order for one row and for three)."""
    n, k = 8, (1 << 24) + 128
    _, args = make_weights(kind, n, k, seed=11)
    x = randn_x(3, k, seed=12)
    y = S.skinny_mm(x, *args)
    assert torch.equal(S.skinny_mm(x[1:2].contiguous(), *args), y[1:2])
    check_against_oracle(y, x, oracle_weights(kind, args))


def test_exact_fixture():
    """Tiny operands whose exact bf16 products are committed (tests/golden/skinny_kat.json): the kernel's fp32
    accumulation may move a result by at most one bf16 step from the exactly rounded value."""
    cases = json.loads((Path(__file__).resolve().parent / "golden" / "skinny_kat.json").read_text())["cases"]
    for c in cases:
        x = torch.tensor(c["x"], dtype=torch.bfloat16, device="cuda")
        w = torch.tensor(c["w"], dtype=torch.bfloat16, device="cuda")
        y = S.skinny_mm(x, w)
        want = ON.from_bf16_bits(np.array(c["y_bf16_bits"], np.uint16))
        got = y.float().cpu().numpy()
        step = np.abs(want) * 2.0 ** -7 + 1e-30
        assert (np.abs(got - want) <= step).all(), (c["m"], c["n"], c["k"])
        assert (got == want).mean() > 0.9


@pytest.mark.parametrize("kind", KINDS)
def test_inside_a_hip_graph_with_changing_inputs(kind):
    """Captured once, replayed several times with new activations and eager work in between; every replay must
    equal the eager result bitwise."""
    _, args = make_weights(kind, 1024, 2048)
    x = randn_x(4, 2048, seed=0)
    y_eager = S.skinny_mm(x, *args)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        S.skinny_mm(x, *args)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = S.skinny_mm(x, *args)
    for seed in range(4):
        x.copy_(randn_x(4, 2048, seed=100 + seed))
        _ = torch.randn(1000, device="cuda").sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, S.skinny_mm(x, *args)), seed
    assert y_eager.shape == y.shape


def test_gemv_int8_equals_the_one_row_skinny_call():
    """gemv_int8 is the one-row launch of the int8 skinny kernel: bitwise equal to skinny_mm at M = 1."""
    from byteprof_amd.quant.hip_int8 import gemv_int8

    for n, k in ((2048, 2048), (8192, 2048), (129, 640)):
        _, args = make_weights("int8", n, k, seed=n)
        x = randn_x(1, k, seed=k)
        assert torch.equal(gemv_int8(x, *args), S.skinny_mm(x, *args)), (n, k)


def _mf_call(kind, x, args, rb, waves, split, xs):
    from byteprof_amd import _lib

    m, k = x.shape
    n = args[0].shape[0]
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(max(1, split * m * n), dtype=torch.float32, device="cuda")
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[args[1].dtype]) if kind == "int8" else (None, 0)
    rc = _lib.lib().bp_skinny_mf(S._KIND_CODE[kind], x.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), m, n,
                                 k, rb, waves, split, xs, ws.data_ptr(), ws.numel() * 4, _lib.stream_ptr(x.device))
    _lib.check(rc, "bp_skinny_mf")
    return y


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", [(2048, 2048), (100352, 2048), (2048, 8192), (129, 640)])
def test_block_count_and_activation_staging_do_not_change_results(kind, n, k):
    """At one K order (waves, split), the weight blocks per workgroup and whether the activations are staged in LDS
    change nothing, bit for bit, at 1, 5, 9 and 16 rows; every variant matches the oracle."""
    _, args = make_weights(kind, n, k, seed=11)
    w_np = oracle_weights(kind, args) if n * k <= 2048 * 8192 else None
    x = randn_x(16, k, seed=12)
    for waves, split in ((4, 1), (2, 2)):
        for m in (1, 5, 9, 16):
            xm = x[:m].contiguous()
            ref = _mf_call(kind, xm, args, 1, waves, split, 0)
            if w_np is not None and m in (1, 16):
                check_against_oracle(ref, xm, w_np)
            for rb in (1, 2, 4):
                for xs in (0, 1):
                    if S._stage_bytes(kind, m, k, split) < 0 and xs:
                        continue
                    assert torch.equal(_mf_call(kind, xm, args, rb, waves, split, xs), ref), (waves, split, m, rb, xs)


@pytest.mark.parametrize("kind,k", [("bf16", 2048), ("int8", 4096), ("int8", 2048)])
def test_every_configuration_matches_the_oracle(kind, k):
    """Every compiled (weight blocks, waves, split, staging) at 1, 5 and 17 rows against the fp32 reference,
    componentwise (the kernel's whole menu at one shape, N = 192)."""
    import itertools

    _, args = make_weights(kind, 192, k, seed=3)
    wf = args[0].float() if kind == "bf16" else args[0].float() * args[1].float()[:, None]
    bad = []
    for m in (1, 5, 17):
        x = randn_x(m, k, seed=m + 40)
        ref = x.float() @ wf.T
        den = (x.float().abs() @ wf.abs().T).clamp(min=1e-30)
        for rb, waves, split, xs in itertools.product((1, 2, 4), (1, 2, 4, 8), (1, 2, 3, 4), (0, 1)):
            if not S._supported(kind, m, rb, waves, xs) or (xs and S._stage_bytes(kind, m, k, split) < 0):
                continue
            y = _mf_call(kind, x, args, rb, waves, split, xs)
            err = float(((y.float() - ref).abs() / den).max())
            if err > 4e-3:
                bad.append((m, rb, waves, split, xs, err))
    assert not bad, bad[:10]


# (N, K, rows, waves, split): launches whose waves have exactly 4, 8 or 16 K segments (the straight-line kernels),
# with full and partial last row blocks
FIXED_PLANS = [(2048, 2048, 8, 4, 1), (6144, 2048, 8, 2, 1), (2050, 2048, 16, 8, 1), (1000, 8192, 8, 8, 1),
               (1000, 8192, 32, 4, 2), (300, 4096, 8, 2, 4), (520, 2048, 8, 1, 1)]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k,rows,waves,split", FIXED_PLANS)
def test_straight_line_kernel_equals_the_general_loop(kind, n, k, rows, waves, split):
    """A launch whose waves all have 4, 8 or 16 segments runs the straight-line kernel of that count; with
    BP_XS_GENERAL the same plan runs the general segment loop. Same segments in the same order: equal bit for bit,
    with and without the LDS-staged activations, at 1..33 rows; and within the oracle's tolerance."""
    from byteprof_amd import _lib

    L = _lib.lib()
    _, args = make_weights(kind, n, k, seed=n + k + waves)
    w_np = oracle_weights(kind, args)
    x = randn_x(33, k, seed=3)
    kc = S._KIND_CODE[kind]
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[args[1].dtype]) if kind == "int8" else (None, 0)
    rb = rows // 8
    fixed_seen = False
    for m in (1, 2, 5, 9, 16, 33):
        xm = x[:m].contiguous()
        ws = torch.empty(max(1, split * m * n), dtype=torch.float32, device="cuda")
        outs = []
        for xs in (0, S.XS_GENERAL, S.XS_STAGE, S.XS_STAGE | S.XS_GENERAL):
            if xs & S.XS_STAGE and (m > 16 or S._stage_bytes(kind, m, k, split) < 0):
                continue
            r = rb if m <= 16 else min(rb, 2)
            y = torch.full((m, n), 7.0, dtype=torch.bfloat16, device="cuda")
            _lib.check(L.bp_skinny_mf(kc, xm.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), m, n, k, r, waves,
                                      split, xs, ws.data_ptr(), ws.numel() * 4, _lib.stream_ptr(xm.device)), "mf")
            outs.append(y)
            fixed_seen |= S.segments_per_wave(kind, k, waves, split, xs) > 0
        torch.cuda.synchronize()
        for y in outs[1:]:
            assert torch.equal(y.view(torch.int16), outs[0].view(torch.int16)), (m, kind, n, k)
        check_against_oracle(outs[0], xm, w_np)
    # bf16 covers 4 / 8 / 16 segments per wave over these plans, int8 4 / 8 / 16 (the others run the general loop)
    assert fixed_seen == (S.segments_per_wave(kind, k, waves, split) > 0)
