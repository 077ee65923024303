"""GPU parity of the activation prologue of the matrix-core skinny kernel (bp_skinny_mf_pro, skinny.prologue_mm).

  - BP_PRO_NORM equals the separate decode norm launch (bp_decode_norm_residual[_rows]: bf16(residual + bf16(gamma *
    rmsnorm(x)))) followed by the plain skinny launch, bit for bit, for the transformed rows (xout) and for the
    products, with and without a residual, at 1, 2 and 3 rows, bf16 and int8 weights, plain and SiLU epilogues;
  - BP_PRO_UNIT_RMS: the transformed rows are the oracle's unit-RMS renormalisation (oracle.linear_set.unit_rms,
    float64) within one bf16 rounding, and the products equal skinny_mm of those rows bit for bit and the oracle
    within the skinny gates;
  - launches that cannot stage their whole rows (more than 16 rows, more than 32 KiB of rows, K not a multiple of
    the segment, unaligned rows) are refused before anything runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd import _lib
from byteprof_amd.optim import skinny as S
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import linear_set as OL
from tests.helpers import check_against_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _norm_rows(x, gamma, residual, eps):
    """The separate decode norm launch over the rows of x."""
    L = _lib.lib()
    out = torch.empty_like(x)
    rows, n = x.shape
    rc = L.bp_decode_norm_residual_rows(x.data_ptr(), gamma.data_ptr(), _lib.ptr(residual), out.data_ptr(), n, eps,
                                        rows, _lib.stream_ptr(x.device))
    _lib.check(rc, "bp_decode_norm_residual_rows")
    return out


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("with_residual", [True, False])
def test_norm_prologue_equals_norm_launch_then_skinny(kind, m, with_residual):
    """1..4 rows: the staged rows in one pass of registers; 5 and 8 (four waves): the rest by LDS loads; gamma and
    the residual rows in LDS beside them (up to 80 KiB in all: 8 rows of 2048 take 68 KiB)."""
    g = _gen(10 + m)
    n, k, eps = 2048, 2048, 1e-6
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = (w, None) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    x = (torch.randn(m, k, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    res = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16) if with_residual else None
    xn = _norm_rows(x, gamma, res, eps)
    want = S.skinny_mm(xn, *[a for a in args if a is not None])
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    xout = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(x, args[0], args[1], out, S.PRO_NORM, gamma=gamma, residual=res, xout=xout, eps=eps)
    torch.cuda.synchronize()
    assert torch.equal(xout, xn)
    assert torch.equal(out, want)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("n,m", [(100352, 1), (2048, 1), (2048, 2), (2048, 5), (6144, 8)])
def test_two_norm_prologue_equals_norm_launch_then_norm_prologue(kind, n, m):
    """gamma2: the last post-feed-forward norm (+ residual) and the final norm in the LM head's launch equal the
    norm launch followed by the one-norm prologue launch, bit for bit (xout: the rows between the two norms)."""
    g = _gen(30 + m)
    k, eps = 2048, 1e-6
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = (w, None) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    x = (torch.randn(m, k, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    gamma2 = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    res = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    xn = _norm_rows(x, gamma, res, eps)
    want = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(xn, args[0], args[1], want, S.PRO_NORM, gamma=gamma2, eps=eps)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    xout = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(x, args[0], args[1], out, S.PRO_NORM, gamma=gamma, residual=res, xout=xout, eps=eps, gamma2=gamma2)
    torch.cuda.synchronize()
    assert torch.equal(xout, xn)
    assert torch.equal(out, want)
    # the final norm itself against the separate norm launch of xn
    ref = S.skinny_mm(_norm_rows(xn, gamma2, None, eps), *[a for a in args if a is not None])
    assert torch.equal(out, ref)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("with_residual,with_gamma2", [(True, True), (True, False), (False, True), (False, False)])
def test_norm_prologue_at_k8192_two_rows(kind, with_residual, with_gamma2):
    """K = 8192 at two rows: the staged rows take 32 KiB; gamma, the residual rows and gamma2 (16 KiB per row or
    vector) join them in LDS while the total stays within 80 KiB, and are otherwise read from memory (residual +
    gamma2: 96 KiB). Both ways equal the separate norm launch(es) followed by the plain launch, bit for bit."""
    g = _gen(40 + 2 * with_residual + with_gamma2)
    n, k, m, eps = 2048, 8192, 2, 1e-6
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = (w, None) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    x = (torch.randn(m, k, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    gamma2 = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16) if with_gamma2 else None
    res = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16) if with_residual else None
    xn = _norm_rows(x, gamma, res, eps)
    xm = _norm_rows(xn, gamma2, None, eps) if with_gamma2 else xn
    want = S.skinny_mm(xm, *[a for a in args if a is not None])
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    xout = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(x, args[0], args[1], out, S.PRO_NORM, gamma=gamma, residual=res, xout=xout, eps=eps, gamma2=gamma2)
    torch.cuda.synchronize()
    assert torch.equal(xout, xn)
    assert torch.equal(out, want)
    # three rows of 8192 do not fit the 32 KiB stage: refused before anything is enqueued
    x3 = torch.zeros(3, k, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError):
        S.prologue_mm(x3, args[0], args[1], torch.empty(3, n, dtype=torch.bfloat16, device=DEV), S.PRO_NORM,
                      gamma=gamma, eps=eps)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_norm_prologue_with_the_silu_epilogue(kind):
    """The fused norm before the interleaved gate|up projection equals norm launch + bp_skinny_mf_silu."""
    g = _gen(20)
    f, k, eps = 8192, 2048, 1e-6
    w = (torch.randn(2 * f, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = (w, None) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    x = torch.randn(1, k, generator=g, device=DEV).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    res = torch.randn(1, k, generator=g, device=DEV).to(torch.bfloat16)
    xn = _norm_rows(x, gamma, res, eps)
    rb, waves, split, xs = S._resolve(kind, 2 * f, k, 1, None)
    assert split == 1
    want = torch.empty(1, f, dtype=torch.bfloat16, device=DEV)
    L = _lib.lib()
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[args[1].dtype]) if kind == "int8" else (None, 0)
    _lib.check(L.bp_skinny_mf_silu(S._KIND_CODE[kind], xn.data_ptr(), args[0].data_ptr(), sc, sdt, want.data_ptr(), 1,
                                   f, k, rb, waves, xs, _lib.stream_ptr(x.device)), "bp_skinny_mf_silu")
    out = torch.empty(1, f, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(x, args[0], args[1], out, S.PRO_NORM, gamma=gamma, residual=res, eps=eps, silu=True)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
@pytest.mark.parametrize("n,k", [(2048, 2048), (6144, 2048), (2048, 8192), (100352, 2048)])
def test_unit_rms_prologue_matches_the_oracle(kind, n, k):
    g = _gen(30)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = (w, None) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    x = (torch.randn(1, k, generator=g, device=DEV) * 7.0).to(torch.bfloat16)
    out = torch.empty(1, n, dtype=torch.bfloat16, device=DEV)
    xout = torch.empty(1, k, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(x, args[0], args[1], out, S.PRO_UNIT_RMS, xout=xout)
    torch.cuda.synchronize()
    want_x = OL.unit_rms(x.float().cpu().numpy()[0])
    got_x = xout.float().cpu().numpy()[0]
    # within one bf16 rounding of the float64 renormalisation
    assert np.all(np.abs(got_x - want_x) <= np.abs(want_x) * 2.0 ** -7 + 1e-30)
    assert torch.equal(out, S.skinny_mm(xout, *[a for a in args if a is not None]))
    wo = w.float().cpu().numpy() if kind == "bf16" else (args[0].float() * args[1].float()[:, None]).cpu().numpy()
    check_against_oracle(out, xout, wo)


def test_unit_rms_of_a_zero_row_is_the_row():
    w = torch.ones(2048, 2048, dtype=torch.bfloat16, device=DEV)
    x = torch.zeros(1, 2048, dtype=torch.bfloat16, device=DEV)
    out = torch.full((1, 2048), 5.0, dtype=torch.bfloat16, device=DEV)
    S.prologue_mm(x, w, None, out, S.PRO_UNIT_RMS)
    torch.cuda.synchronize()
    assert not out.any()
    with pytest.raises(ValueError):  # a plan that splits K cannot renormalise whole rows
        S.prologue_mm(x, w[:64], None, out[:, :64], S.PRO_UNIT_RMS, cfg=(8, 4, 2))


def test_prologue_refusals():
    L = _lib.lib()
    w = torch.zeros(64, 2048, dtype=torch.bfloat16, device=DEV)
    x = torch.zeros(17, 2048, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(17, 64, dtype=torch.bfloat16, device=DEV)
    st = _lib.stream_ptr(x.device)

    def call(pro, m=1, k=2048, xp=None):
        return L.bp_skinny_mf_pro(0, xp or x.data_ptr(), w.data_ptr(), None, 0, y.data_ptr(), m, 64, k, 1, 4, 0, pro, st)

    import ctypes
    assert call(None) == -1
    assert call(ctypes.byref(S.BpPrologue(3, 0.0, None, None, None))) == -1       # unknown kind
    assert call(ctypes.byref(S.BpPrologue(2, 0.0, None, None, None))) == -1       # norm without gamma
    unit = ctypes.byref(S.BpPrologue(1, 0.0, None, None, None))
    assert call(unit, m=17) == -2                                                   # more than 16 rows
    assert call(unit, m=16) == -2                                                   # 16 x 2048 rows: 64 KiB of LDS
    assert call(unit, m=9) == -2                                                    # 9 x 2048 rows: 36 KiB of LDS
    assert call(unit, k=2000) == -2                                                 # K not a multiple of the segment
    assert call(unit, xp=x.data_ptr() + 2) == -2                                    # unaligned rows
    g = torch.ones(2050, dtype=torch.bfloat16, device=DEV)
    assert call(ctypes.byref(S.BpPrologue(2, 1e-6, g.data_ptr() + 2, None, None))) == -1  # unaligned gamma
    assert call(ctypes.byref(S.BpPrologue(1, 0.0, None, None, None, g.data_ptr()))) == -1  # gamma2 without a norm
    assert call(ctypes.byref(S.BpPrologue(2, 1e-6, g.data_ptr(), None, None, g.data_ptr() + 2))) == -1  # unaligned
    torch.cuda.synchronize()


def _int4_pro(x, args, out, tile, waves, silu, kind, gamma=None, res=None, xout=None, gamma2=None, eps=1e-6):
    packed, scale, zero = args
    p = S.BpPrologue(kind, eps, _lib.ptr(gamma), _lib.ptr(res), _lib.ptr(xout), _lib.ptr(gamma2))
    m, k = x.shape
    return _lib.lib().bp_skinny_int4_pro(x.data_ptr(), packed.data_ptr(), scale.data_ptr(), _lib.TORCH_DT[scale.dtype],
                                         zero.data_ptr(), out.data_ptr(), m, out.shape[1], k, tile, waves, int(silu),
                                         __import__("ctypes").byref(p), _lib.stream_ptr(x.device))


def _int4_plain(x, args, n, tile, waves, silu):
    """bp_skinny_int4 (split 1), then bp_decode_silu_mul_rows for the gate|up product."""
    L = _lib.lib()
    packed, scale, zero = args
    m, k = x.shape
    y = torch.empty(m, 2 * n if silu else n, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_skinny_int4(x.data_ptr(), packed.data_ptr(), scale.data_ptr(), _lib.TORCH_DT[scale.dtype],
                                zero.data_ptr(), y.data_ptr(), m, y.shape[1], k, tile, waves, 1, None, 0,
                                _lib.stream_ptr(x.device)), "bp_skinny_int4")
    if not silu:
        return y
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_decode_silu_mul_rows(y.data_ptr(), out.data_ptr(), n, m, 1, _lib.stream_ptr(x.device)), "silu")
    return out


@pytest.mark.parametrize("tile", [16, 32, 64])
@pytest.mark.parametrize("k,m", [(2048, 1), (384, 1), (8192, 1), (2048, 3), (2048, 7), (384, 8)])
def test_int4_norm_prologue_equals_norm_launch_then_int4(tile, k, m):
    """bp_skinny_int4_pro: the rows, gamma, the residual rows and gamma2 staged in LDS, then the int4 matrix-core
    kernel; equal bit for bit to the norm launch(es) followed by bp_skinny_int4 at the same tile rows and waves (with
    the SiLU epilogue: then bp_decode_silu_mul_rows), with and without the residual and gamma2; K 384 leaves a
    partial 512-element staging chunk, K 8192 at one row and 2048 at seven rows fill the 64 KiB; xout receives the
    rows before the second norm."""
    g = _gen(60 + tile + k + m)
    n, eps = 1000, 1e-6
    w = (torch.randn(2 * n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = S.quantize_int4(w, tile)
    x = (torch.randn(m, k, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    gamma2 = (1.0 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    res = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    print(f"\n[int4 pro] tile={tile} k={k} m={m}", flush=True)
    for r, g2 in ((res, None), (None, None), (res, gamma2), (None, gamma2)):
        xn = _norm_rows(x, gamma, r, eps)
        xm = _norm_rows(xn, g2, None, eps) if g2 is not None else xn
        for silu in (False, True):
            nn = n if silu else 2 * n
            for waves in (1, 4):
                want = _int4_plain(xm, args, nn, tile, waves, silu)
                out = torch.full((m, nn), float("nan"), dtype=torch.bfloat16, device=DEV)
                xout = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
                _lib.check(_int4_pro(x, args, out, tile, waves, silu, S.PRO_NORM, gamma, r, xout, g2, eps),
                           "bp_skinny_int4_pro")
                torch.cuda.synchronize()
                assert torch.equal(xout, xn), (r is None, g2 is None, silu, waves)
                assert torch.equal(out, want), (r is None, g2 is None, silu, waves)


def test_int4_unit_rms_prologue_and_refusals():
    """BP_PRO_UNIT_RMS with int4 weights: xout within one bf16 rounding of x / rms(x) (float64), the product equal
    to bp_skinny_int4 of xout bit for bit; nine rows, fp16 scales, staging past 64 KiB of LDS and an xout
    overlapping x are refused before anything runs."""
    g = _gen(77)
    n, k = 2048, 2048
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    args = S.quantize_int4(w, 32)
    x = (torch.randn(1, k, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    out = torch.empty(1, n, dtype=torch.bfloat16, device=DEV)
    xout = torch.empty(1, k, dtype=torch.bfloat16, device=DEV)
    _lib.check(_int4_pro(x, args, out, 32, 4, False, S.PRO_UNIT_RMS, xout=xout), "bp_skinny_int4_pro")
    torch.cuda.synchronize()
    xd = x.double()
    want_rows = xd / xd.pow(2).mean().sqrt()
    assert ((xout.double() - want_rows).abs() <= want_rows.abs() * 2.0 ** -8 + 1e-30).all()
    assert torch.equal(out, _int4_plain(xout, args, n, 32, 4, False))
    gamma = torch.ones(k, dtype=torch.bfloat16, device=DEV)
    x9 = torch.zeros(9, k, dtype=torch.bfloat16, device=DEV)
    assert _int4_pro(x9, args, torch.empty(9, n, dtype=torch.bfloat16, device=DEV), 32, 4, False, S.PRO_NORM,
                     gamma) == _lib.BP_E_UNSUPPORTED
    a16 = (args[0], args[1].to(torch.float16), args[2])
    assert _int4_pro(x, a16, out, 32, 4, False, S.PRO_NORM, gamma) == _lib.BP_E_UNSUPPORTED
    wk = (torch.randn(256, 8320, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    xk = torch.zeros(1, 8320, dtype=torch.bfloat16, device=DEV)
    gk = torch.ones(8320, dtype=torch.bfloat16, device=DEV)
    assert _int4_pro(xk, S.quantize_int4(wk, 16), torch.empty(1, 256, dtype=torch.bfloat16, device=DEV), 16, 4,
                     False, S.PRO_NORM, gk) == _lib.BP_E_UNSUPPORTED
    big = torch.zeros(2, k, dtype=torch.bfloat16, device=DEV)
    assert _int4_pro(big[:1], args, out, 32, 4, False, S.PRO_NORM, gamma, xout=big[:1]) == _lib.BP_E_INVALID_ARG
    torch.cuda.synchronize()
