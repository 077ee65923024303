"""The drop-in modules on the GPU: `apply_quantization(..., kernel="skinny")` on a toy OLMo-shaped model, the
kernel and dequantized paths of SkinnyLinear, SkinnyLinear inside a HIP graph with bias, fp32 activations, and the
skinny int8 and default int8 modules sharing identical quantized weights. Mirrors byteprof
tests/test_skinny_integration.py:66-175."""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from tests.test_host import _Toy

pytestmark = pytest.mark.gpu


def _toy(seed=0):
    torch.manual_seed(seed)
    return _Toy().to("cuda", torch.bfloat16)


@pytest.mark.parametrize("scheme", ["bf16_wo", "int8_wo"])
def test_apply_quantization_with_the_skinny_kernel_swaps_selected_linears(scheme):
    from byteprof_amd.optim.skinny_linear import SkinnyLinear
    from byteprof_amd.quant.integrate import apply_quantization

    m = _toy()
    stats = apply_quantization(m, "blocks", scheme, 128, None, None, "skinny")
    assert stats["kernel"] == "skinny" and stats["n_linears"] == 14
    assert sum(isinstance(x, SkinnyLinear) for x in m.modules()) == 14 and isinstance(m.lm_head, nn.Linear)
    ref = _toy()
    for rows in (1, 5, 64, 100):  # kernel, kernel, kernel (chunked), dequantize fallback
        xr = torch.randn(rows, 256, device="cuda", dtype=torch.bfloat16)
        a = m.model.layers[0].self_attn["q_proj"](xr).float()
        b = ref.model.layers[0].self_attn["q_proj"](xr).float()
        assert a.shape == b.shape == (rows, 256)
        tol = {"bf16_wo": 1e-2, "int8_wo": 0.1}[scheme]
        assert (a - b).abs().max() < tol * b.abs().max()
    assert m.model.layers[0].self_attn["q_proj"](torch.empty(0, 256, device="cuda", dtype=torch.bfloat16)).shape == (0, 256)
    assert m.model.layers[0].self_attn["q_proj"].weight.dtype == torch.bfloat16


def test_skinny_int8_uses_the_same_quantized_weights_as_the_default_int8():
    from byteprof_amd.optim.skinny_linear import SkinnyLinear
    from byteprof_amd.quant.integrate import Int8Linear

    lin = nn.Linear(512, 128, bias=False, dtype=torch.bfloat16, device="cuda")
    a, b = Int8Linear(lin), SkinnyLinear(lin, "int8_wo")
    assert torch.equal(a.q, b.q) and torch.equal(a.scale, b.scale)
    x = torch.randn(1, 512, device="cuda", dtype=torch.bfloat16)
    assert (a(x).float() - b(x).float()).abs().max() < 0.02 * a(x).float().abs().max()


def test_skinny_linear_inside_a_hip_graph_with_bias():
    from byteprof_amd.optim.skinny_linear import SkinnyLinear

    lin = nn.Linear(256, 96, bias=True, dtype=torch.bfloat16, device="cuda")
    for scheme in ("bf16_wo", "int8_wo"):
        m = SkinnyLinear(lin, scheme)
        x = torch.randn(3, 1, 256, device="cuda", dtype=torch.bfloat16)
        eager = m(x)
        with torch.inference_mode():
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                m(x)
            torch.cuda.current_stream().wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                y = m(x)
            for _ in range(3):
                x.copy_(torch.randn_like(x))
                g.replay()
                torch.cuda.synchronize()
                assert torch.equal(y, m(x))
        assert eager.shape == (3, 1, 96)


@pytest.mark.parametrize("scheme", ["int8_wo"])
def test_fp32_activations_use_the_dequantized_weights(scheme):
    from byteprof_amd.optim.skinny_linear import SkinnyLinear

    lin = nn.Linear(256, 64, bias=False, dtype=torch.float32, device="cuda")
    m = SkinnyLinear(lin, scheme)
    x = torch.randn(3, 256, device="cuda", dtype=torch.float32)
    y = m(x)
    assert y.dtype == torch.float32
    assert torch.allclose(y, x @ m.dequantized(torch.float32).T, atol=1e-5, rtol=1e-5)
    assert (y - lin(x)).abs().max() < 0.1 * lin(x).abs().max()


def test_native_library_is_what_runs():
    """The kernel path loads libbyteprof_amd.so from the package directory (no fallback module exists)."""
    from byteprof_amd import _lib

    _lib.lib()
    maps = open("/proc/self/maps", encoding="utf-8").read()
    assert str(_lib.LIB_PATH) in maps
