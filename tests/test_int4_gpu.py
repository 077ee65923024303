"""int4 group-128 skinny kernel (skinny_int4.hip) on the GPU against the CPU oracle: every M = 1..33 on the
reference's real and odd shapes, tile heights, configurations, bitwise row independence, the sentinel out-of-bounds
check, scale dtypes, graph capture and SkinnyLinear int4_wo. Mirrors byteprof tests/test_skinny.py:71-149 for the
int4 kind."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd.optim import skinny as S
from oracle import skinny as OS
from tests.helpers import check_against_oracle, randn_x

pytestmark = pytest.mark.gpu

REAL = [(2048, 2048), (8192, 2048), (2048, 8192), (1024, 2048), (2816, 2048), (2048, 2816)]
ODD = [(37, 256), (1, 128), (50, 384), (129, 640)]


def make_int4(n: int, k: int, seed: int = 0, tile_rows: int = 32, scale_dtype=None):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    packed, scale, zero = S.quantize_int4(w, tile_rows)
    if scale_dtype is not None:
        scale = scale.to(scale_dtype)
    w_np = OS.dequantize_int4(packed.cpu().numpy(), scale.float().cpu().numpy(), zero.float().cpu().numpy())
    return (packed, scale, zero), w_np


@pytest.mark.parametrize("n,k", REAL + ODD)
def test_matches_the_oracle_for_every_m(n, k):
    print(f"\n[int4] n={n} k={k}", flush=True)
    args, w_np = make_int4(n, k, seed=n + k)
    x = randn_x(33, k, seed=7)
    worst = (0.0, 0.0)
    for m in range(1, 34):
        y = S.skinny_mm(x[:m].contiguous(), *args)
        assert y.shape == (m, n) and y.dtype == torch.bfloat16
        worst = max(worst, check_against_oracle(y, x[:m], w_np))
    print("worst componentwise / normwise", worst)


@pytest.mark.parametrize("tile_rows", [16, 64])
@pytest.mark.parametrize("n,k", [(37, 256), (2048, 2048), (129, 640)])
def test_tile_heights(tile_rows, n, k):
    args, w_np = make_int4(n, k, seed=3, tile_rows=tile_rows)
    assert args[0].shape[2] == tile_rows
    x = randn_x(16, k, seed=1)
    for m in (1, 7, 16):
        check_against_oracle(S.skinny_mm(x[:m].contiguous(), *args), x[:m], w_np)


@pytest.mark.parametrize("tile_rows", [16, 32, 64])
@pytest.mark.parametrize("scale_dtype", [None, torch.float16, torch.float32])
def test_silu_epilogue_equals_the_product_then_silu_mul(tile_rows, scale_dtype):
    """bp_skinny_int4_silu on an interleaved gate|up weight: bit for bit bp_skinny_int4 (same tile rows and waves)
    followed by bp_decode_silu_mul_rows, for 1..16 rows and a ragged last tile; the sums checked against the
    oracle."""
    from byteprof_amd import _lib

    L = _lib.lib()
    for ffn, k in ((512, 1024), (1000, 512)):
        args, w_np = make_int4(2 * ffn, k, seed=ffn, tile_rows=tile_rows, scale_dtype=scale_dtype)
        packed, scale, zero = args
        for waves in (1, 4):
            for m in (1, 5, 16):
                x = randn_x(m, k, seed=m + ffn)
                gu = torch.empty(m, 2 * ffn, dtype=torch.bfloat16, device="cuda")
                _lib.check(L.bp_skinny_int4(x.data_ptr(), packed.data_ptr(), scale.data_ptr(),
                                            _lib.TORCH_DT[scale.dtype], zero.data_ptr(), gu.data_ptr(), m, 2 * ffn, k,
                                            tile_rows, waves, 1, None, 0, _lib.stream_ptr(x.device)), "int4")
                ref = torch.empty(m, ffn, dtype=torch.bfloat16, device="cuda")
                _lib.check(L.bp_decode_silu_mul_rows(gu.data_ptr(), ref.data_ptr(), ffn, m, 1,
                                                     _lib.stream_ptr(x.device)), "silu")
                out = torch.full((m, ffn), float("nan"), dtype=torch.bfloat16, device="cuda")
                _lib.check(L.bp_skinny_int4_silu(x.data_ptr(), packed.data_ptr(), scale.data_ptr(),
                                                 _lib.TORCH_DT[scale.dtype], zero.data_ptr(), out.data_ptr(), m, ffn,
                                                 k, tile_rows, waves, _lib.stream_ptr(x.device)), "int4 silu")
                assert torch.equal(out, ref), (ffn, k, waves, m)
                if m == 16:
                    check_against_oracle(gu, x, w_np)


def test_k_past_the_buffer_range_takes_the_valu_kernel():
    """K >= 2^24: the matrix-core kernel reads its activations through one buffer resource (under 2^31 bytes at 16
    rows), so such K takes the VALU kernel at every row count (the same K order for one row and for three)."""
    n, k = 16, (1 << 24) + 128
    args, w_np = make_int4(n, k, seed=21, tile_rows=16)
    x = randn_x(3, k, seed=22)
    y = S.skinny_mm(x, *args)
    assert torch.equal(S.skinny_mm(x[1:2].contiguous(), *args), y[1:2])
    check_against_oracle(y, x, w_np)


@pytest.mark.parametrize("cfg", [(1, 1), (2, 1), (4, 1), (8, 1), (2, 3), (8, 2), (32, 128, 4, 3, 5)])
def test_configurations_match(cfg):
    args, w_np = make_int4(192, 2048, seed=5)
    for m in (1, 5, 16, 17):
        x = randn_x(m, 2048, seed=m)
        check_against_oracle(S.skinny_mm(x, *args, cfg=cfg), x, w_np)


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_scale_dtypes(scale_dtype):
    args, w_np = make_int4(300, 1024, seed=8, scale_dtype=scale_dtype)
    x = randn_x(4, 1024, seed=2)
    check_against_oracle(S.skinny_mm(x, *args), x, w_np)


@pytest.mark.parametrize("n,k", [(2048, 2048), (129, 640), (2048, 8192)])
def test_rows_do_not_depend_on_the_other_rows(n, k):
    """One int4 kernel serves 1..16 rows with one K order: row i is bitwise the same for every M (2048 x 8192: the
    activations staged in LDS up to 3 rows, loaded with the weights past that)."""
    args, _ = make_int4(n, k, seed=4)
    x = randn_x(33, k, seed=3)
    full16 = S.skinny_mm(x[:16].contiguous(), *args)
    for m in (1, 2, 3, 5, 9, 15):
        assert torch.equal(S.skinny_mm(x[:m].contiguous(), *args), full16[:m]), m
    full33 = S.skinny_mm(x, *args)
    assert torch.equal(full33[:16], full16)
    assert torch.equal(S.skinny_mm(x[16:19].contiguous(), *args), full33[16:19])


@pytest.mark.parametrize("m", [1, 3, 17])
def test_kernel_writes_only_the_output_block(m):
    n, k = 70, 384
    args, w_np = make_int4(n, k, seed=1)
    x = randn_x(m, k, seed=8)
    flat = torch.full((m * n + 4096,), 777.0, device="cuda", dtype=torch.bfloat16)
    out = flat[:m * n].view(m, n)
    S.skinny_mm(x, *args, out=out)
    assert torch.equal(flat[m * n:], torch.full_like(flat[m * n:], 777.0))
    assert not (out == 777.0).any()
    check_against_oracle(out, x, w_np)


def test_unaligned_activations_and_empty_inputs():
    args, w_np = make_int4(64, 256, seed=2)
    buf = randn_x(3 * 256 + 1, 1, seed=5).reshape(-1)
    x = buf[1:].view(3, 256)  # 2-byte offset: the host copies it to an aligned buffer
    check_against_oracle(S.skinny_mm(x, *args), x, w_np)
    assert S.skinny_mm(torch.empty(0, 256, device="cuda", dtype=torch.bfloat16), *args).shape == (0, 64)


def test_graph_replays_match_eager():
    args, _ = make_int4(2048, 2048, seed=6)
    x = randn_x(5, 2048, seed=3)
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


def test_skinny_linear_int4_scheme():
    from byteprof_amd.optim.skinny_linear import SkinnyLinear

    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 300, bias=True, dtype=torch.bfloat16, device="cuda")
    m = SkinnyLinear(lin, "int4_wo")
    x = torch.randn(2, 3, 512, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        y = m(x)
        ref = x.float() @ m.dequantized(torch.float32).T + lin.bias.float()
    assert y.shape == (2, 3, 300) and m.q.shape[2] == S.int4_tile_rows(300, 512)
    assert float((y.float() - ref).abs().max() / ref.abs().max()) < 1e-2
