"""bp_skinny_mf_static (split-K partials in the library's fixed device array: no workspace argument, no allocation)
against bp_skinny_mf with a caller workspace, through the C ABI: equal bit for bit on two calls in a row on one
stream, the second with a smaller input. (Its refusal of partials larger than the array runs on the CPU:
tests/test_abi.py.)"""

from __future__ import annotations

import pytest
import torch

from byteprof_amd import _lib
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operands(kind, m, n, k, g):
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    if kind == "bf16":
        return x, w, None, 0
    q, s = quantize_rowwise_int8(w, torch.float16)
    return x, q, s, _lib.TORCH_DT[s.dtype]


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_static_scratch_entry_equals_the_workspace_entry(kind):
    L = _lib.lib()
    kc = 0 if kind == "bf16" else 1
    g = torch.Generator(device=DEV).manual_seed(5)
    assert L.bp_skinny_mf_static_bytes() == 8 << 20
    calls = [(16, 8192, 8192, 8), (3, 2048, 4096, 4)]  # 4 MiB of partials, then 96 KiB
    outs = []
    for m, n, k, split in calls:
        print(f"\n[no-alloc] {kind} M={m} N={n} K={k} split={split}", flush=True)
        x, w, sc, sdt = _operands(kind, m, n, k, g)
        st = _lib.stream_ptr(x.device)
        ws = torch.empty(split * m * n, dtype=torch.float32, device=DEV)
        want = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        _lib.check(L.bp_skinny_mf(kc, x.data_ptr(), w.data_ptr(), _lib.ptr(sc), sdt, want.data_ptr(), m, n, k, 1, 4,
                                  split, 0, ws.data_ptr(), ws.numel() * 4, st), "bp_skinny_mf")
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        _lib.check(L.bp_skinny_mf_static(kc, x.data_ptr(), w.data_ptr(), _lib.ptr(sc), sdt, got.data_ptr(), m, n, k,
                                         1, 4, split, 0, st), "bp_skinny_mf_static")
        outs.append((got, want, (x, w, sc, ws)))
    torch.cuda.synchronize()
    for got, want, _ in outs:
        assert torch.equal(got, want)
