"""Fused int8 weight-only product on the GPU against the dequantize-then-matmul oracle: the one-row gemv_int8 on
real and odd shapes and other block configurations, Int8Linear for every row count with bias, empty inputs,
fp16 scales, graph capture. Mirrors byteprof tests/test_quant_int8.py:19-123."""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from byteprof_amd.quant.hip_int8 import gemv_int8, quantize_rowwise_int8
from oracle import numerics as ON
from oracle import skinny as OS
from tests.helpers import randn_x

pytestmark = pytest.mark.gpu


def _oracle(x, q, s, bias=None):
    y = OS.matmul(x.float().cpu().numpy(), OS.dequantize("int8", q.cpu().numpy(), s.float().cpu().numpy()))
    if bias is not None:
        y = y + bias.detach().float().cpu().numpy()[None, :]
    return y


def _close(y, ref):
    """max |y - ref| <= 0.01 max |ref| + 1e-3 (tests/test_quant_int8.py:53-56)."""
    assert y.dtype == torch.bfloat16
    err = float(abs(y.detach().float().cpu().numpy() - ref).max())
    assert err <= 0.01 * float(abs(ref).max()) + 1e-3, err


REAL_SHAPES = [(1024, 2048), (2048, 2048), (2816, 2048), (2048, 2816), (8192, 2048), (2048, 8192)]


@pytest.mark.parametrize("n,k", REAL_SHAPES)
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
def test_gemv_real_shapes_batch_one(n, k, scale_dtype):
    g = torch.Generator(device="cuda").manual_seed(n * 7 + k)
    q, s = quantize_rowwise_int8((torch.randn(n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16),
                                 scale_dtype)
    x = randn_x(1, k, seed=1)
    _close(gemv_int8(x, q, s), _oracle(x, q, s))


@pytest.mark.parametrize("n,k", [(37, 1000), (1, 8), (3, 129), (1025, 2049), (16, 2047), (7, 5000), (24, 128)])
def test_gemv_odd_sizes_not_multiples_of_block(n, k):
    g = torch.Generator(device="cuda").manual_seed(n + k)
    q, s = quantize_rowwise_int8((torch.randn(n, k, generator=g, device="cuda") * 0.05).to(torch.bfloat16))
    x = randn_x(1, k, seed=2)
    ref = _oracle(x, q, s)
    _close(gemv_int8(x, q, s), ref)
    for cfg in ((1, 256, 1), (8, 1024, 8), (4, 2), (16, 4)):  # reference (BN, BK, warps) and native (rows, waves)
        _close(gemv_int8(x, q, s, cfg), ref)


@pytest.mark.parametrize("m", [1, 2, 5, 33, 300])
@pytest.mark.parametrize("n,k,bias", [(2048, 2048, True), (2816, 2048, False), (37, 1000, True)])
def test_int8linear_all_row_counts_vs_the_oracle(m, n, k, bias):
    from byteprof_amd.quant.integrate import Int8Linear

    torch.manual_seed(m + n)
    lin = nn.Linear(k, n, bias=bias, dtype=torch.bfloat16, device="cuda")
    mod = Int8Linear(lin)
    x = torch.randn(m, 1, k, device="cuda", dtype=torch.bfloat16)
    y = mod(x)
    assert y.shape == (m, 1, n)
    _close(y.reshape(m, n), _oracle(x.reshape(m, k), mod.q, mod.scale, lin.bias if bias else None))


def test_int8linear_single_row_and_batch_paths_agree_with_bias():
    from byteprof_amd.quant.integrate import Int8Linear

    lin = nn.Linear(256, 64, bias=True, dtype=torch.bfloat16, device="cuda")
    m = Int8Linear(lin)
    assert m.weight.dtype == torch.bfloat16 and m.weight.numel() == 0
    x = torch.randn(3, 1, 256, device="cuda", dtype=torch.bfloat16)
    batch = m(x)
    single = torch.cat([m(x[i:i + 1]) for i in range(3)])
    assert batch.shape == single.shape == (3, 1, 64)
    assert (batch.float() - single.float()).abs().max() < 0.05
    assert (batch.float() - lin(x).float()).abs().max() < 0.1


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_int8linear_one_row_of_any_float_dtype_takes_the_kernel(dtype, monkeypatch):
    """One fp32 or fp16 row goes through the fused int8 product, as in the reference, whose GEMV reads x as fp32
    (integrate.py:40-42, triton_int8.py:24): never through the dequantized weight; the result is in x's dtype and
    within the int8 tolerance of the oracle on the unrounded activations."""
    from byteprof_amd.quant.integrate import Int8Linear

    torch.manual_seed(11)
    n, k = 2048, 2048
    lin = nn.Linear(k, n, bias=True, dtype=dtype, device="cuda")
    mod = Int8Linear(lin)

    def refuse(_dtype):
        raise AssertionError("a one-row GPU call dequantized the weight")

    monkeypatch.setattr(mod, "dequantized", refuse)
    x = torch.randn(1, 1, k, device="cuda", dtype=dtype)
    with torch.no_grad():
        y = mod(x)
    assert y.shape == (1, 1, n) and y.dtype == dtype
    ref = _oracle(x.reshape(1, k), mod.q, mod.scale, lin.bias)
    err = float(abs(y.reshape(1, n).float().cpu().numpy() - ref).max())
    assert err <= 0.01 * float(abs(ref).max()) + 1e-3, err
    out = torch.empty(1, n, dtype=dtype, device="cuda")
    assert gemv_int8(x.reshape(1, k), mod.q, mod.scale, out=out) is out
    ref_nb = _oracle(x.reshape(1, k), mod.q, mod.scale)
    err = float(abs(out.float().cpu().numpy() - ref_nb).max())
    assert err <= 0.01 * float(abs(ref_nb).max()) + 1e-3, err


def test_int8linear_empty_input():
    from byteprof_amd.quant.integrate import Int8Linear

    mod = Int8Linear(nn.Linear(256, 64, bias=True, dtype=torch.bfloat16, device="cuda"))
    for shape in ((0, 256), (0, 1, 256)):
        y = mod(torch.empty(*shape, device="cuda", dtype=torch.bfloat16))
        assert y.shape == (*shape[:-1], 64) and y.numel() == 0


def test_gemv_inside_a_hip_graph_matches_eager():
    q, s = quantize_rowwise_int8((torch.randn(2048, 2048, device="cuda") * 0.02).to(torch.bfloat16))
    x = randn_x(1, 2048, seed=3)
    gemv_int8(x, q, s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = gemv_int8(x, q, s)
    for seed in range(3):
        x.copy_(randn_x(1, 2048, seed=10 + seed))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, gemv_int8(x, q, s))


def test_quantizer_on_the_gpu_matches_the_oracle_bit_for_bit():
    w = (torch.randn(256, 1024, device="cuda") * 0.02).to(torch.bfloat16)
    q, s = quantize_rowwise_int8(w)
    oq, os_ = OS.quantize_rowwise_int8(w.float().cpu().numpy(), "bf16")
    assert (q.cpu().numpy() == oq).all() and (s.float().cpu().numpy() == os_).all()
    assert ON.normwise_error(OS.dequantize("int8", oq, os_), w.float().cpu().numpy()) < 1e-2
