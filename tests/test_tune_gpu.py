"""The tuner on the GPU (byteprof_amd/tune.py, the role of byteprof tools/skinny_tune.py:30-93): on a small shape it
returns one K order for every row bucket and, per bucket, a plan that runs and matches the oracle; the int4 tuner
returns a plan whose launches match the oracle too."""

from __future__ import annotations

import pytest
import torch

from byteprof_amd import tune as T
from byteprof_amd.optim import skinny as S
from tests.helpers import check_against_oracle, make_weights, oracle_weights, randn_x

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_tuned_plan_is_one_k_order_and_matches_the_oracle(kind):
    n, k = 512, 1024
    print(f"\n[tune] {kind} {n}x{k}", flush=True)
    e = T.tune_shape(kind, n, k, DEV, log=lambda m: None)
    assert e["waves"] in (1, 2, 4, 8) and 1 <= e["split"] <= k // S.k_segment(kind)
    assert set(e["rb"]) == set(e["xs"]) == {"1", "8", "16", "32", "64"}
    assert {"1", "4", "8", "16", "32", "64"} <= set(e["us"]) and all(v > 0 for v in e["us"].values())
    _, args = make_weights(kind, n, k, seed=3)
    w_np = oracle_weights(kind, args)
    from byteprof_amd import _lib

    L = _lib.lib()
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[args[1].dtype]) if kind == "int8" else (None, 0)
    for m, bucket in ((1, "1"), (8, "8"), (16, "16"), (33, "64")):
        x = randn_x(m, k, seed=m)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        split = e["split"]
        ws = torch.empty(max(1, split * m * n), dtype=torch.float32, device=DEV)
        _lib.check(L.bp_skinny_mf(S._KIND_CODE[kind], x.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), m, n, k,
                                  int(e["rb"][bucket]), e["waves"], split, int(e["xs"][bucket]), ws.data_ptr(),
                                  ws.numel() * 4, _lib.stream_ptr(DEV)), "bp_skinny_mf")
        check_against_oracle(y, x, w_np)
    # the norm-prologue plans (rb_pro) at the same K order: equal bit for bit to the plain launch on the normed rows
    assert set(e.get("rb_pro", {})) <= {"1", "8"}
    gamma = (1 + 0.1 * torch.randn(k, generator=torch.Generator(device=DEV).manual_seed(5), device=DEV)).to(
        torch.bfloat16)
    for bucket, m in (("1", 1), ("8", 4)):
        if bucket not in e.get("rb_pro", {}):
            continue
        x = randn_x(m, k, seed=10 + m)
        xn = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        S.prologue_mm(x, args[0], args[1] if kind == "int8" else None, y, S.PRO_NORM, gamma=gamma, xout=xn, eps=1e-6,
                      cfg=(8 * int(e["rb_pro"][bucket]), e["waves"], 1))
        want = S.skinny_mm(xn, *args, cfg=(8 * int(e["rb"][bucket]), e["waves"], 1))
        assert torch.equal(y, want)


def test_int4_tuned_plan_matches_the_oracle():
    n, k = 512, 1024
    e = T.tune_int4(n, k, DEV, log=lambda m: None)
    assert e["waves"] in (1, 2, 4, 8) and 1 <= e["split"] <= k // S.GROUP and e["tile_rows"] in S.INT4_TILES
    assert set(e["tiles"]) == {str(t) for t in S.INT4_TILES}
    w = (torch.randn(n, k, generator=torch.Generator(device=DEV).manual_seed(4), device=DEV) * 0.02).to(torch.bfloat16)
    packed, scale, zero = S.quantize_int4(w, e["tile_rows"])
    w_np = S.dequantize("int4", packed, scale, zero).cpu().numpy()
    for m in (1, 4, 16):
        x = randn_x(m, k, seed=m)
        check_against_oracle(S.skinny_mm(x, packed, scale, zero, cfg=(e["waves"], e["split"])), x, w_np)
