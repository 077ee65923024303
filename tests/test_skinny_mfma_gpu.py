"""Matrix-core skinny kernels (skinny_mfma.hip) on the GPU against the CPU oracle: every compiled configuration on
ragged shapes, the routed configurations on the decode shapes at the verify widths, bitwise row independence,
the sentinel out-of-bounds check, argmax parity over the LM head, graph capture, argument checks."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from byteprof_amd import _lib
from byteprof_amd.optim import skinny as S
from tests.helpers import check_against_oracle, make_weights, oracle_weights, randn_x

pytestmark = pytest.mark.gpu

KINDS = ["bf16", "int8"]
BLOCK_ROWS = (16, 32, 64)
WAVES = (1, 2, 4, 8)
DEPTHS = (1, 2)


def _mfma(kind, x, args, block_rows, waves, depth, split, n):
    y = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=x.device)
    S.launch_mfma(kind, x, args[0], args[1] if kind == "int8" else None, y, block_rows, waves, depth, split)
    return y


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("depth", DEPTHS)
def test_every_configuration_matches_the_oracle(kind, depth):
    n, k = 70, 1024  # N not a multiple of any block, 4 (int8) / 8 (bf16) K steps
    print(f"\n[mfma] kind={kind} depth={depth} n={n} k={k}", flush=True)
    _, args = make_weights(kind, n, k, seed=5)
    w_np = oracle_weights(kind, args)
    x = randn_x(16, k, seed=11)
    for br in BLOCK_ROWS:
        for waves in WAVES:
            for split in (1, 3):
                for m in (1, 5, 16):
                    y = _mfma(kind, x[:m].contiguous(), args, br, waves, depth, split, n)
                    check_against_oracle(y, x[:m], w_np)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("depth", S.STAGED_DEPTHS)
def test_staged_configurations_match_the_oracle(kind, depth):
    """The LDS-staged variants (16-row blocks; depth 3 each wave owns whole blocks, depth 4 the waves share them):
    every wave count, K of one to six 1 KiB steps, K slices of one workgroup up to 2048 (larger K needs split),
    ragged N, 1..16 rows."""
    for n, k in ((70, 1024), (33, 3072), (1000, 6144)):
        print(f"\n[mfma-staged] kind={kind} depth={depth} n={n} k={k}", flush=True)
        _, args = make_weights(kind, n, k, seed=n + k)
        w_np = oracle_weights(kind, args)
        x = randn_x(16, k, seed=13)
        for waves in (1, 2, 4):
            splits = {S.staged_split(kind, k, 1, waves, depth), S.staged_split(kind, k, 3, waves, depth)} - {None}
            assert splits
            for split in sorted(splits):
                for m in (1, 5, 16):
                    y = _mfma(kind, x[:m].contiguous(), args, 16, waves, depth, split, n)
                    check_against_oracle(y, x[:m], w_np)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("depth", S.STAGED_DEPTHS)
def test_staged_rows_do_not_depend_on_the_other_rows(kind, depth):
    n, k = 300, 4096
    _, args = make_weights(kind, n, k, seed=19)
    x = randn_x(16, k, seed=7)
    split = S.staged_split(kind, k, 1, 4, depth)
    full = _mfma(kind, x, args, 16, 4, depth, split, n)
    for m in (1, 3, 8, 15):
        assert torch.equal(_mfma(kind, x[:m].contiguous(), args, 16, 4, depth, split, n), full[:m]), m
    if depth == 3:  # each wave adds a block's steps in K order, whatever the number of waves
        assert torch.equal(_mfma(kind, x, args, 16, 1, depth, split, n), full)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", [(2048, 2048), (8192, 2048), (2048, 8192), (6144, 2048), (16384, 2048),
                                 (100352, 2048)])
def test_verify_widths_match_the_oracle(kind, n, k):
    """skinny_mm at 5..16 rows takes the matrix-core path on the decode shapes (K a multiple of the step)."""
    print(f"\n[mfma] kind={kind} n={n} k={k}", flush=True)
    assert S.mfma_cfg(kind, n, k) is not None
    _, args = make_weights(kind, n, k, seed=n ^ k)
    w_np = oracle_weights(kind, args)
    x = randn_x(16, k, seed=2)
    for m in (5, 8, 16):
        check_against_oracle(S.skinny_mm(x[:m].contiguous(), *args), x[:m], w_np)


@pytest.mark.parametrize("kind", KINDS)
def test_rows_do_not_depend_on_the_other_rows(kind):
    n, k = 512, 2048
    _, args = make_weights(kind, n, k, seed=9)
    x = randn_x(16, k, seed=4)
    for br, waves, depth, split in ((16, 4, 2, 1), (64, 8, 1, 2)):
        full = _mfma(kind, x, args, br, waves, depth, split, n)
        for m in (1, 2, 7, 8, 15):
            assert torch.equal(_mfma(kind, x[:m].contiguous(), args, br, waves, depth, split, n), full[:m]), m
        # the workgroup shape (block rows, prefetch depth) does not change the K order either
        other = _mfma(kind, x, args, 32 if br != 32 else 16, waves, 3 - depth, split, n)
        assert torch.equal(other, full)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [1, 9, 16])
def test_kernel_writes_only_the_output_block(kind, m):
    n, k = 70, 512 if kind == "bf16" else 768
    _, args = make_weights(kind, n, k, seed=1)
    w_np = oracle_weights(kind, args)
    x = randn_x(m, k, seed=8)
    flat = torch.full((m * n + 4096,), 777.0, device="cuda", dtype=torch.bfloat16)
    out = flat[:m * n].view(m, n)
    S.launch_mfma(kind, x, args[0], args[1] if kind == "int8" else None, out, 64, 2, 2, 1)
    assert torch.equal(flat[m * n:], torch.full_like(flat[m * n:], 777.0))
    assert not (out == 777.0).any()
    check_against_oracle(out, x, w_np)


@pytest.mark.parametrize("kind", KINDS)
def test_lm_head_argmax_matches_at_sixteen_rows(kind):
    """Greedy verify over the 100352-row head: every row's argmax is the oracle's, unless the oracle's top two are
    closer than one bf16 step of the maximum (then either is accepted)."""
    n, k = 100352, 2048
    _, args = make_weights(kind, n, k, seed=3)
    w_np = oracle_weights(kind, args)
    x = randn_x(16, k, seed=21)
    y = S.skinny_mm(x, *args).float().cpu().numpy()
    ref = x.float().cpu().numpy().astype(np.float64) @ w_np.astype(np.float64).T
    for r in range(16):
        top2 = np.sort(ref[r])[-2:]
        gap = top2[1] - top2[0]
        got, want = int(np.argmax(y[r])), int(np.argmax(ref[r]))
        if got != want:
            assert gap < abs(top2[1]) * 2.0 ** -7, (r, got, want, gap)


@pytest.mark.parametrize("kind", KINDS)
def test_graph_replays_match_eager(kind):
    n, k = 2048, 2048
    _, args = make_weights(kind, n, k, seed=6)
    x = randn_x(12, k, seed=3)
    eager = S.skinny_mm(x, *args)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        S.skinny_mm(x, *args, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        S.skinny_mm(x, *args, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_argument_checks():
    L = _lib.lib()
    w = torch.zeros(32, 200, device="cuda", dtype=torch.bfloat16)
    x = torch.zeros(2, 200, device="cuda", dtype=torch.bfloat16)
    y = torch.empty(2, 32, device="cuda", dtype=torch.bfloat16)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    call = lambda m, k, br=16, waves=1, depth=1: L.bp_skinny_mfma_bf16(  # noqa: E731
        x.data_ptr(), w.data_ptr(), y.data_ptr(), m, 32, k, br, waves, depth, 1, None, 0, stream)
    assert call(2, 200) == -2          # K not a multiple of the 128-element step
    assert call(17, 128) == -1         # more than 16 activation rows
    assert call(2, 128, br=24) == -2   # block rows not a multiple of 16
    assert call(2, 128, br=128) == -2  # not compiled
    assert call(2, 128, waves=3) == -2
    assert call(2, 128, depth=3) == -2           # the staged variants need K a multiple of 512 (bf16)
    assert call(2, 512, br=32, depth=4) == -2    # and 16-row blocks
    assert call(2, 512, waves=8, depth=3) == -2  # at most 4 waves
    assert call(2, 1536, waves=2, depth=4) == -2  # 3 steps: not a multiple or divisor of 2 sharing waves
    assert call(2, 128, depth=5) == -2
    assert L.bp_skinny_mfma_config_supported(0, 16, 4, 4) == 1
    assert L.bp_skinny_mfma_config_supported(1, 16, 2, 3) == 1
    assert L.bp_skinny_mfma_config_supported(0, 32, 4, 3) == 0
    assert L.bp_skinny_mfma_config_supported(0, 64, 8, 2) == 1
    assert L.bp_skinny_mfma_config_supported(1, 48, 8, 2) == 0
    torch.cuda.synchronize()
