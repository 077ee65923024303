"""Row groups over one staged copy of the activation rows (BP_XS_ROWS2 / BP_XS_ROWS4 with BP_XS_STAGE, 9..16 rows):
each row group's waves split K as the plain kernel's do, so every output row equals the plain kernel's bit for bit
(the K order depends only on (K, waves, split), byteprof tests/test_skinny.py:74-87 asks it across row counts), for
every compiled (rb, waves), ragged N included; and the oracle agrees."""

from __future__ import annotations

import pytest
import torch

from byteprof_amd import _lib
from byteprof_amd.optim import skinny as S
from tests.helpers import check_against_oracle, make_weights, oracle_weights, randn_x

pytestmark = pytest.mark.gpu


def _launch(kind, args, x, n, rb, waves, xs):
    m, k = x.shape
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=x.device)
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[args[1].dtype]) if kind == "int8" else (None, 0)
    _lib.check(_lib.lib().bp_skinny_mf(S._KIND_CODE[kind], x.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), m,
                                       n, k, rb, waves, 1, xs, None, 0, _lib.stream_ptr(x.device)),
               "bp_skinny_mf")
    return y


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("n,k", [(2048, 2048), (1000, 2048), (8200, 1024), (300, 1536)])
def test_row_groups_equal_the_plain_kernel_bit_for_bit(kind, n, k):
    print(f"\n[rows] {kind} n={n} k={k}", flush=True)
    _, args = make_weights(kind, n, k, seed=n + k)
    ran = 0
    for m in (9, 13, 16):
        x = randn_x(m, k, seed=m + k)
        for waves in (2, 4, 8):
            if not S._supported(kind, m, 1, waves, 0):
                continue
            ref = _launch(kind, args, x, n, 1, waves, 0)
            for rows in (S.XS_ROWS2, S.XS_ROWS4):
                xs = S.XS_STAGE | rows
                if S._stage_bytes(kind, m, k, 1, xs) < 0:
                    continue
                for rb in (1, 2, 4):
                    if not S._supported(kind, m, rb, waves, xs):
                        continue
                    y = _launch(kind, args, x, n, rb, waves, xs)
                    assert torch.equal(y, ref), (m, waves, rb, rows)
                    ran += 1
        if m == 16:
            check_against_oracle(ref, x, oracle_weights(kind, args))
    assert ran > 0  # the menu holds row-group kernels for these shapes


def test_row_group_flags_are_ignored_outside_their_plans(monkeypatch):
    """At 8 rows or fewer, without staging, or past the 64 KiB staging limit, a plan with row-group flags resolves
    to a plan without them (skinny_mm never launches an uncompiled row-group kernel)."""
    assert S._stage_bytes("bf16", 16, 2048, 1, S.XS_STAGE | S.XS_ROWS2) == 16 * 2048 * 2
    assert S._stage_bytes("bf16", 16, 2048, 1) < 0  # over the 32 KiB of a plain staged launch
    assert S._stage_bytes("bf16", 16, 4096, 1, S.XS_STAGE | S.XS_ROWS4) < 0  # over 64 KiB
    for m, k, xs in ((4, 2048, S.XS_STAGE | S.XS_ROWS2), (16, 2048, S.XS_ROWS4), (16, 4096, S.XS_STAGE | S.XS_ROWS4)):
        monkeypatch.setattr(S, "_table_plan", lambda kind, n, k_, m_, pro=False, xs=xs: (1, 4, 1, xs))
        assert S._resolve("bf16", 2048, k, m, None)[3] & S.XS_ROWS == 0, (m, k, xs)
    monkeypatch.setattr(S, "_table_plan", lambda kind, n, k_, m_, pro=False: (2, 4, 1, S.XS_STAGE | S.XS_ROWS4))
    assert S._resolve("bf16", 2048, 2048, 16, None)[3] == S.XS_STAGE | S.XS_ROWS4


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("ffn", [1024, 500])
def test_row_groups_with_the_silu_epilogue_equal_the_plain_kernel(kind, ffn):
    """The gate|up launch of a verify round (interleaved gate / up rows, SiLU product epilogue) with row groups: bit
    for bit the plain launch's outputs."""
    print(f"\n[rows silu] {kind} ffn={ffn}", flush=True)
    k = 2048
    _, args = make_weights(kind, 2 * ffn, k, seed=ffn)
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[args[1].dtype]) if kind == "int8" else (None, 0)

    def silu(x, rb, waves, xs):
        out = torch.full((x.shape[0], ffn), float("nan"), dtype=torch.bfloat16, device=x.device)
        _lib.check(_lib.lib().bp_skinny_mf_silu(S._KIND_CODE[kind], x.data_ptr(), args[0].data_ptr(), sc, sdt,
                                                out.data_ptr(), x.shape[0], ffn, k, rb, waves, xs,
                                                _lib.stream_ptr(x.device)), "bp_skinny_mf_silu")
        return out

    ran = 0
    for m in (9, 16):
        x = randn_x(m, k, seed=m)
        for waves in (2, 4):
            ref = silu(x, 1, waves, 0)
            assert not torch.isnan(ref.float()).any()
            for rows in (S.XS_ROWS2, S.XS_ROWS4):
                for rb in (1, 2, 4):
                    if S._supported(kind, m, rb, waves, S.XS_STAGE | rows):
                        assert torch.equal(silu(x, rb, waves, S.XS_STAGE | rows), ref), (m, waves, rb, rows)
                        ran += 1
    assert ran > 0
