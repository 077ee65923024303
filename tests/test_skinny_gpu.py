"""Skinny matmul kernels on the GPU against the CPU oracle: every M = 1..33 on the reference's real and odd shapes,
empty inputs and chunking, split-K and other tile configurations, bitwise row independence, validation, the
sentinel out-of-bounds check, unaligned inputs, graph capture. Mirrors byteprof tests/test_skinny.py:71-149."""

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
@pytest.mark.parametrize("n,k", [(2048, 2048), (2048, 8192), (129, 640)])
def test_rows_do_not_depend_on_the_other_rows(kind, n, k):
    """Output row i is bitwise the same whatever the number of rows in the call, within each kernel family: the VALU
    kernels (1..4 rows: one K order) and the matrix-core kernels (5..16 rows) (byteprof tests/test_skinny.py:114-121,
    whose single M <= 16 bucket is split where the arithmetic unit changes)."""
    _, args = make_weights(kind, n, k)
    x = randn_x(33, k, seed=3)
    full4 = S.skinny_mm(x[:4].contiguous(), *args)
    for m in (1, 2, 3):
        assert torch.equal(S.skinny_mm(x[:m].contiguous(), *args), full4[:m]), m
    full16 = S.skinny_mm(x[:16].contiguous(), *args)
    full33 = S.skinny_mm(x, *args)
    assert torch.equal(full33[:16], full16)
    for m in (5, 8, 9, 15):
        assert torch.equal(S.skinny_mm(x[:m].contiguous(), *args), full16[:m]), m
    assert torch.equal(S.skinny_mm(x[16:32].contiguous(), *args), full33[16:32])
    assert torch.equal(S.skinny_mm(x[32:33].contiguous(), *args), full33[32:33])


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
