"""The benchmark workloads at their full sizes on the GPU. Here the oracle is the reference's own fp32
formulation (`x.float() @ dequantize(...).T` on the device, byteprof tests/test_skinny.py:38 and
tests/test_quant_int8.py:48-50) plus size-independent properties, because the CPU oracle is too slow at
2048 x 100352 x 16:
  - the single 8192 x 2048 linear at M = 1;
  - the decode-step sweep M in {1,2,4,8,16} x K in {2048, 8192} x N in {2048, 8192, 100352} (normwise <= 1e-2);
  - greedy argmax parity over the 100352-wide LM head (ties closer than one bf16 step are reported, not hidden);
  - the int8 set with fp16 scales at M in {1, 4, 16};
  - linearity in x (y(a x1 + x2) against a y(x1) + y(x2) within the rounding bound) and a checksum of the output
    against (W^T u) . x for a random u, computed from the CPU oracle in float64 on the same operands."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd.optim import skinny as S
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from tests.helpers import check_against_oracle, make_weights, normwise, oracle_weights, randn_x, torch_reference

pytestmark = pytest.mark.gpu


def unit_rms(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (xf / xf.pow(2).mean(dim=-1, keepdim=True).sqrt()).to(torch.bfloat16)


def test_single_linear_8192x2048_m1():
    _, args = make_weights("bf16", 8192, 2048, seed=1)
    x = randn_x(1, 2048, seed=1)
    y = S.skinny_mm(x, *args)
    comp, norm = check_against_oracle(y, x, oracle_weights("bf16", args))
    print(f"\n[C1] componentwise {comp:.3e} normwise {norm:.3e}")


@pytest.mark.parametrize("n", [2048, 8192, 100352])
@pytest.mark.parametrize("k", [2048, 8192])
def test_sweep_cells(n, k):
    print(f"\n[sweep] n={n} k={k}", flush=True)
    _, args = make_weights("bf16", n, k, seed=n + k)
    w32 = args[0].float()
    x = unit_rms(randn_x(16, k, seed=k))
    full = S.skinny_mm(x, *args)
    scale = x.float().abs() @ w32.abs().T  # the componentwise bound's denominator (sum of absolute terms)
    for m in (1, 2, 4, 8, 16):
        y = S.skinny_mm(x[:m].contiguous(), *args)
        ref = torch_reference(x[:m], w32)
        err = normwise(y, ref)
        assert err < 1e-2, (m, err)
        comp = float(((y.float() - ref).abs() / scale[:m].clamp(min=1e-30)).max())
        assert comp < 4e-3, (m, comp)
        assert torch.equal(y, full[:m])  # one K order for every row count
    del w32


def test_lm_head_argmax_parity():
    """argmax of the bf16 kernel output against argmax of the bf16-rounded fp32 reference (first index on ties,
    as torch.argmax). A mismatch is accepted only where the reference's top-2 gap is below one bf16 step."""
    _, args = make_weights("bf16", 100352, 2048, seed=5)
    w32 = args[0].float()
    flips = []
    for seed in range(8):
        x = unit_rms(randn_x(16, 2048, seed=100 + seed))
        y = S.skinny_mm(x, *args)
        ref = torch_reference(x, w32)
        want = ref.to(torch.bfloat16).float().argmax(dim=1)
        got = y.float().argmax(dim=1)
        top2 = ref.topk(2, dim=1).values
        gap = (top2[:, 0] - top2[:, 1])
        ulp = top2[:, 0].abs() * 2.0 ** -8
        for r in torch.nonzero(got != want).flatten().tolist():
            flips.append((seed, r, float(gap[r]), float(ulp[r])))
            assert gap[r] <= 2 * ulp[r], (seed, r, float(gap[r]))
    print(f"\n[head] argmax flips within one bf16 step: {flips}")
    assert len(flips) <= 2


@pytest.mark.parametrize("n,k", [(2048, 2048), (8192, 2048), (2048, 8192), (100352, 2048)])
def test_int8_set_shapes_with_fp16_scales(n, k):
    g = torch.Generator(device="cuda").manual_seed(n ^ k)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    q, s = quantize_rowwise_int8(w, torch.float16)
    assert s.dtype == torch.float16
    deq = q.float() * s.float()[:, None]
    x = unit_rms(randn_x(16, k, seed=3))
    full = {4: S.skinny_mm(x[:4].contiguous(), q, s), 16: S.skinny_mm(x, q, s)}
    for m in (1, 4, 16):
        y = S.skinny_mm(x[:m].contiguous(), q, s)
        assert normwise(y, torch_reference(x[:m], deq)) < 1e-2
        assert torch.equal(y, full[4 if m <= 4 else 16][:m])
        assert normwise(y, torch_reference(x[:m], w.float())) < 5e-2  # quantization error only


def test_linearity_and_checksum_on_the_lm_head():
    _, args = make_weights("bf16", 100352, 2048, seed=9)
    x1 = randn_x(1, 2048, seed=1)
    x2 = randn_x(1, 2048, seed=2)
    xs = (x1.float() + x2.float()).to(torch.bfloat16)
    y1, y2, ys = (S.skinny_mm(x, *args).float() for x in (x1, x2, xs))
    # y(x1 + x2) vs y(x1) + y(x2): differences only from the bf16 roundings of xs and of the three outputs
    assert normwise(ys, y1 + y2) < 3e-2
    # checksum: u . y == (W^T u) . x, with W^T u from the CPU oracle in float64
    u = np.random.default_rng(0).standard_normal(100352)
    wtu = args[0].float().cpu().numpy().astype(np.float64).T @ u
    lhs = float(u @ y1.cpu().numpy()[0])
    rhs = float(wtu @ x1.float().cpu().numpy()[0])
    bound = float(np.abs(u) @ np.abs(y1.cpu().numpy()[0])) * 2.0 ** -8
    assert abs(lhs - rhs) < bound, (lhs, rhs, bound)
