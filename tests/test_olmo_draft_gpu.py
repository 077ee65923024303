"""GPU parity of the drafting (verify) path of the decode loop (optim/olmo_draft.py, OlmoDecoder.verify, the *_rows
decode kernels and bp_draft_verify_next).

  - every *_rows kernel equals the one-row kernel called at each row's position, bit for bit, and the fused
    rope_attention (one row) and rope_attention_rows equal qk_rope_cache(_rows) + attention(_rows) bit for bit;
  - the round's end on the device: accepted length, the row tokens, the next round's first token and position;
  - a verify pass of s rows, teacher-forced, against the oracle's sequential decode steps (the decode gate), every s
    from 1 to 9;
  - the drafting loop on the OLMo-2-1B shape produces the plain graph loop's tokens exactly: with no drafts and with
    the oracle drafter at 2..4, up to 9 and up to 16 rows per round (every kernel of a row computes it as the
    one-token step does, bit for bit, whatever the row count).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd import _lib
from byteprof_amd.optim import olmo as OG
from byteprof_amd.optim import olmo_draft as OD
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import numerics as ON
from oracle import olmo as OO
from tests.test_olmo_gpu import GATE, SMALL, _bf16, _np, _ocfg, _small_decoder

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROPE_CFGS = {"d64": SMALL, "d128": OG.OlmoConfig(hidden=2048, ffn=512, layers=1, heads=16, vocab=512, max_len=512)}


def _st():
    return _lib.stream_ptr(torch.device(DEV))


@pytest.mark.parametrize("shape", ["d64", "d128"])
def test_rope_cache_and_attention_rows_equal_the_one_row_calls(shape):
    """qk_rope_cache_rows / attention_rows over 6 rows at base 40 against the one-row kernels at positions 40..45;
    the fused rope_attention against qk_rope_cache + attention at one position; all bit for bit."""
    cfg = ROPE_CFGS[shape]
    oc = _ocfg(cfg)
    L = _lib.lib()
    H, D, S, base = cfg.hidden, cfg.head_dim, 6, 40
    rng = np.random.default_rng(3)
    qkv = _bf16(ON.bf16_round(rng.standard_normal((S, 3 * H)).astype(np.float32)))
    qw, kw = (_bf16(ON.bf16_round(1 + 0.1 * rng.standard_normal(H).astype(np.float32))) for _ in range(2))
    cache0 = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    inv = torch.from_numpy(OO.inv_freq(oc)).to(DEV)
    kc_a, vc_a, kc_b, vc_b = (_bf16(cache0) for _ in range(4))
    q_a, q_b = (torch.empty(S, H, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    o_a, o_b = (torch.empty(S, H, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    pos = torch.tensor([base], dtype=torch.int64, device=DEV)
    args = (cfg.heads, D, cfg.max_len, cfg.eps)
    _lib.check(L.bp_decode_qk_rope_cache_rows(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                              pos.data_ptr(), q_a.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(), *args,
                                              S, _st()), "rows")
    _lib.check(L.bp_decode_attention_rows(q_a.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(), pos.data_ptr(),
                                          o_a.data_ptr(), cfg.heads, D, cfg.max_len, D ** -0.5, S, _st()), "rows")
    for r in range(S):
        p = torch.tensor([base + r], dtype=torch.int64, device=DEV)
        _lib.check(L.bp_decode_qk_rope_cache(qkv[r].data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                             p.data_ptr(), q_b[r].data_ptr(), kc_b.data_ptr(), vc_b.data_ptr(),
                                             *args, _st()), "one")
        _lib.check(L.bp_decode_attention(q_b[r].data_ptr(), kc_b.data_ptr(), vc_b.data_ptr(), p.data_ptr(),
                                         o_b[r].data_ptr(), cfg.heads, D, cfg.max_len, D ** -0.5, _st()), "one")
    torch.cuda.synchronize()
    for a, b in ((q_a, q_b), (kc_a, kc_b), (vc_a, vc_b), (o_a, o_b)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # the fused kernel at the last position, on a fresh copy of the caches before that position was written
    kc_c, vc_c = _bf16(cache0), _bf16(cache0)
    kc_c[:, :base + S - 1] = kc_b[:, :base + S - 1]
    vc_c[:, :base + S - 1] = vc_b[:, :base + S - 1]
    o_c = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    p = torch.tensor([base + S - 1], dtype=torch.int64, device=DEV)
    _lib.check(L.bp_decode_rope_attention(qkv[S - 1].data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                          p.data_ptr(), kc_c.data_ptr(), vc_c.data_ptr(), o_c.data_ptr(), cfg.heads,
                                          D, cfg.max_len, cfg.eps, D ** -0.5, _st()), "fused")
    torch.cuda.synchronize()
    assert torch.equal(o_c.view(torch.int16), o_b[S - 1].view(torch.int16))
    assert torch.equal(kc_c.view(torch.int16), kc_b.view(torch.int16))


ROWS_CFGS = dict(ROPE_CFGS, d256=OG.OlmoConfig(hidden=512, ffn=512, layers=1, heads=2, vocab=512, max_len=300),
                 d8=OG.OlmoConfig(hidden=64, ffn=512, layers=1, heads=8, vocab=512, max_len=600))


@pytest.mark.parametrize("shape,rows,base", [("d64", 1, 0), ("d64", 2, 0), ("d64", 9, 37), ("d64", 16, 100),
                                             ("d128", 2, 40), ("d128", 9, 40), ("d128", 16, 500),
                                             ("d256", 5, 296), ("d8", 9, 3), ("d128", 9, 506)])
def test_fused_rope_attention_rows_equal_the_two_launch_rows(shape, rows, base):
    """rope_attention_rows (norms, RoPE, cache write and attention of every row in one launch) against
    qk_rope_cache_rows + attention_rows on the same inputs: outputs and both caches equal bit for bit, also where
    the last rows fall beyond the cache (base 296 + 5 > 300, 506 + 9 > 512)."""
    cfg = ROWS_CFGS[shape]
    oc = _ocfg(cfg)
    L = _lib.lib()
    H, D = cfg.hidden, cfg.head_dim
    rng = np.random.default_rng(rows * 1000 + base)
    qkv = _bf16(ON.bf16_round(rng.standard_normal((rows, 3 * H)).astype(np.float32)))
    qw, kw = (_bf16(ON.bf16_round(1 + 0.1 * rng.standard_normal(H).astype(np.float32))) for _ in range(2))
    cache0 = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    inv = torch.from_numpy(OO.inv_freq(oc)).to(DEV)
    kc_a, vc_a, kc_b, vc_b = (_bf16(cache0) for _ in range(4))
    q_a = torch.empty(rows, H, dtype=torch.bfloat16, device=DEV)
    o_a, o_b = (torch.full((rows, H), 7.0, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    pos = torch.tensor([base], dtype=torch.int64, device=DEV)
    _lib.check(L.bp_decode_qk_rope_cache_rows(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                              pos.data_ptr(), q_a.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(),
                                              cfg.heads, D, cfg.max_len, cfg.eps, rows, _st()), "rows")
    _lib.check(L.bp_decode_attention_rows(q_a.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(), pos.data_ptr(),
                                          o_a.data_ptr(), cfg.heads, D, cfg.max_len, D ** -0.5, rows, _st()), "rows")
    _lib.check(L.bp_decode_rope_attention_rows(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                               pos.data_ptr(), kc_b.data_ptr(), vc_b.data_ptr(), o_b.data_ptr(),
                                               cfg.heads, D, rows, cfg.max_len, cfg.eps, D ** -0.5, _st()), "fused")
    torch.cuda.synchronize()
    for a, b in ((o_a, o_b), (kc_a, kc_b), (vc_a, vc_b)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert _lib.lib().bp_decode_rope_attention_rows(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                                    pos.data_ptr(), kc_b.data_ptr(), vc_b.data_ptr(), o_b.data_ptr(),
                                                    cfg.heads, D, 17, cfg.max_len, cfg.eps, D ** -0.5, _st()) != 0


@pytest.mark.parametrize("shape,rows,base", [("d128", 2, 0), ("d128", 4, 8), ("d128", 4, 125), ("d128", 9, 126),
                                             ("d128", 16, 250), ("d64", 3, 5), ("d256", 5, 120), ("d8", 4, 61)])
def test_fused_rows_equal_the_fused_one_row_steps(shape, rows, base):
    """rope_attention_rows over rows at base against rope_attention called at base, base + 1, ... in turn (the
    drafting loop against the one-token loop, directly): outputs and caches equal bit for bit, and a second
    one-row pass over the same inputs gives the same bits (no race in the launch)."""
    cfg = ROWS_CFGS[shape]
    oc = _ocfg(cfg)
    L = _lib.lib()
    H, D = cfg.hidden, cfg.head_dim
    rng = np.random.default_rng(rows * 7 + base)
    qkv = _bf16(ON.bf16_round(rng.standard_normal((rows, 3 * H)).astype(np.float32)))
    qw, kw = (_bf16(ON.bf16_round(1 + 0.1 * rng.standard_normal(H).astype(np.float32))) for _ in range(2))
    cache0 = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    inv = torch.from_numpy(OO.inv_freq(oc)).to(DEV)
    kc_a, vc_a = _bf16(cache0), _bf16(cache0)
    o_a = torch.empty(rows, H, dtype=torch.bfloat16, device=DEV)
    pos = torch.tensor([base], dtype=torch.int64, device=DEV)
    _lib.check(L.bp_decode_rope_attention_rows(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                               pos.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(), o_a.data_ptr(),
                                               cfg.heads, D, rows, cfg.max_len, cfg.eps, D ** -0.5, _st()), "rows")
    outs = []
    for _ in range(2):
        kc_b, vc_b = _bf16(cache0), _bf16(cache0)
        o_b = torch.empty(rows, H, dtype=torch.bfloat16, device=DEV)
        for r in range(rows):
            p = torch.tensor([base + r], dtype=torch.int64, device=DEV)
            _lib.check(L.bp_decode_rope_attention(qkv[r].data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(),
                                                  p.data_ptr(), kc_b.data_ptr(), vc_b.data_ptr(), o_b[r].data_ptr(),
                                                  cfg.heads, D, cfg.max_len, cfg.eps, D ** -0.5, _st()), "one")
        outs.append((o_b, kc_b, vc_b))
    torch.cuda.synchronize()
    for o_b, kc_b, vc_b in outs:
        for r in range(rows):
            assert torch.equal(o_a[r].view(torch.int16), o_b[r].view(torch.int16)), f"row {r}"
        assert torch.equal(kc_a.view(torch.int16), kc_b.view(torch.int16))
        assert torch.equal(vc_a.view(torch.int16), vc_b.view(torch.int16))


@pytest.mark.parametrize("plan", [(1, 4, 0), (2, 2, 0), (4, 8, 0), (1, 4, 1)])
@pytest.mark.parametrize("m", [1, 5, 9, 16])
@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_mf_silu_equals_mf_then_silu_mul(kind, m, plan):
    """The gate|up launch with the SiLU epilogue against the same launch (split 1) followed by silu_mul_rows on the
    interleaved rows: equal bit for bit at 1..16 rows. F = 1000 leaves a partial last block."""
    L = _lib.lib()
    F, K = 1000, 2048
    rb, waves, xs = plan
    rng = np.random.default_rng(m * 7 + waves)
    x = _bf16(ON.bf16_round(rng.standard_normal((m, K)).astype(np.float32)))
    w = _bf16(ON.bf16_round(rng.standard_normal((2 * F, K)).astype(np.float32) * 0.05))
    args = (w,) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[torch.float16]) if kind == "int8" else (None, 0)
    kc = 0 if kind == "bf16" else 1
    out = torch.full((m, F), 3.0, dtype=torch.bfloat16, device=DEV)
    if xs and L.bp_skinny_mf_stage_bytes(kc, m, K, 1) < 0:
        # the activations of this row count do not fit the LDS stage: refused before anything is enqueued
        assert L.bp_skinny_mf_silu(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, out.data_ptr(), m, F, K, rb, waves,
                                   xs, _st()) == -2
        torch.cuda.synchronize()
        assert bool((out == 3.0).all())
        return
    _lib.check(L.bp_skinny_mf_silu(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, out.data_ptr(), m, F, K, rb, waves,
                                   xs, _st()), "mf_silu")
    gu = torch.empty(m, 2 * F, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_skinny_mf(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, gu.data_ptr(), m, 2 * F, K, rb, waves,
                              1, xs, None, 0, _st()), "mf")
    ref = torch.empty(m, F, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_decode_silu_mul_rows(gu.data_ptr(), ref.data_ptr(), F, m, 1, _st()), "silu_mul_rows")
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert L.bp_skinny_mf_silu(kc, x.data_ptr(), w.data_ptr(), sc, sdt, out.data_ptr(), m, F, K, rb, 3, xs,
                               _st()) == -2  # no kernel with 3 waves


@pytest.mark.parametrize("plan", [(1, 4, 2, 0), (2, 8, 2, 0), (1, 4, 4, 1), (4, 2, 3, 0)])
@pytest.mark.parametrize("m", [1, 5, 9, 16])
@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_splitk_norm_residual_equals_reduce_then_norm(kind, m, plan):
    """The down projection of a verify pass: the split-K partials reduced inside the norm launch, against the
    launch with its own reduce followed by norm_residual_rows: equal bit for bit (in place on the residual, as the
    decoder runs it)."""
    L = _lib.lib()
    H, F = 2048, 8192
    rb, waves, split, xs = plan
    rng = np.random.default_rng(m * 11 + waves + split)
    x = _bf16(ON.bf16_round(rng.standard_normal((m, F)).astype(np.float32)))
    w = _bf16(ON.bf16_round(rng.standard_normal((H, F)).astype(np.float32) * 0.02))
    nw = _bf16(ON.bf16_round(1 + 0.1 * rng.standard_normal(H).astype(np.float32)))
    r0 = _bf16(ON.bf16_round(rng.standard_normal((m, H)).astype(np.float32)))
    args = (w,) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)
    sc, sdt = (args[1].data_ptr(), _lib.TORCH_DT[torch.float16]) if kind == "int8" else (None, 0)
    kc = 0 if kind == "bf16" else 1
    ws = torch.empty(split * m * H, dtype=torch.float32, device=DEV)
    ra, rbuf = r0.clone(), r0.clone()
    if xs and L.bp_skinny_mf_stage_bytes(kc, m, F, split) < 0:
        # the activations of this row count do not fit the LDS stage: both launches are refused before anything is
        # enqueued
        assert L.bp_skinny_mf_partials(kc, x.data_ptr(), args[0].data_ptr(), m, H, F, rb, waves, split, xs,
                                       ws.data_ptr(), ws.numel() * 4, _st()) == -2
        y = torch.full((m, H), 3.0, dtype=torch.bfloat16, device=DEV)
        assert L.bp_skinny_mf(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), m, H, F, rb, waves, split,
                              xs, ws.data_ptr(), ws.numel() * 4, _st()) == -2
        torch.cuda.synchronize()
        assert bool((y == 3.0).all())
        return
    _lib.check(L.bp_skinny_mf_partials(kc, x.data_ptr(), args[0].data_ptr(), m, H, F, rb, waves, split, xs,
                                       ws.data_ptr(), ws.numel() * 4, _st()), "partials")
    _lib.check(L.bp_decode_splitk_norm_residual_rows(ws.data_ptr(), split, sc, sdt, nw.data_ptr(), ra.data_ptr(),
                                                     ra.data_ptr(), H, 1e-6, m, _st()), "splitk_norm")
    y = torch.empty(m, H, dtype=torch.bfloat16, device=DEV)
    ws2 = torch.empty_like(ws)
    _lib.check(L.bp_skinny_mf(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), m, H, F, rb, waves, split,
                              xs, ws2.data_ptr(), ws2.numel() * 4, _st()), "mf")
    _lib.check(L.bp_decode_norm_residual_rows(y.data_ptr(), nw.data_ptr(), rbuf.data_ptr(), rbuf.data_ptr(), H, 1e-6,
                                              m, _st()), "norm_rows")
    torch.cuda.synchronize()
    assert torch.equal(ra.view(torch.int16), rbuf.view(torch.int16))
    assert L.bp_skinny_mf_partials(kc, x.data_ptr(), args[0].data_ptr(), m, H, F, rb, waves, 1, xs, ws.data_ptr(),
                                   ws.numel() * 4, _st()) == -2  # partials need split >= 2
    assert L.bp_skinny_mf_partials(kc, x.data_ptr(), args[0].data_ptr(), m, H, F, rb, waves, split, xs,
                                   ws.data_ptr(), 16, _st()) == -3  # workspace too small


def test_norm_silu_embed_argmax_rows_equal_the_one_row_calls():
    L = _lib.lib()
    rng = np.random.default_rng(5)
    S, n, F, V = 7, 2048, 3000, 100352
    x = _bf16(ON.bf16_round(rng.standard_normal((S, n)).astype(np.float32) * 2))
    w = _bf16(ON.bf16_round(1 + 0.1 * rng.standard_normal(n).astype(np.float32)))
    r0 = _bf16(ON.bf16_round(rng.standard_normal((S, n)).astype(np.float32)))
    ra, rb = r0.clone(), r0.clone()
    _lib.check(L.bp_decode_norm_residual_rows(x.data_ptr(), w.data_ptr(), ra.data_ptr(), ra.data_ptr(), n, 1e-6, S,
                                              _st()), "rows")
    for r in range(S):
        _lib.check(L.bp_decode_norm_residual(x[r].data_ptr(), w.data_ptr(), rb[r].data_ptr(), rb[r].data_ptr(), n,
                                             1e-6, _st()), "one")
    gu = _bf16(ON.bf16_round(rng.standard_normal((S, 2 * F)).astype(np.float32) * 3))
    sa, sb, sc = (torch.empty(S, F, dtype=torch.bfloat16, device=DEV) for _ in range(3))
    _lib.check(L.bp_decode_silu_mul_rows(gu.data_ptr(), sa.data_ptr(), F, S, 0, _st()), "rows")
    _lib.check(L.bp_decode_silu_mul_rows(gu.data_ptr(), sc.data_ptr(), F, S, 1, _st()), "rows interleaved")
    for r in range(S):
        _lib.check(L.bp_decode_silu_mul(gu[r].data_ptr(), sb[r].data_ptr(), F, _st()), "one")
    deint = torch.cat([gu[:, 0::2], gu[:, 1::2]], dim=1).contiguous()
    sd = torch.empty(S, F, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_decode_silu_mul_rows(deint.data_ptr(), sd.data_ptr(), F, S, 0, _st()), "rows")
    table = _bf16(ON.bf16_round(rng.standard_normal((600, n)).astype(np.float32)))
    ids = torch.tensor([5, 0, 599, 17, 17, 300, 1], dtype=torch.int64, device=DEV)
    ea = torch.empty(S, n, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_decode_embed_rows(ids.data_ptr(), table.data_ptr(), ea.data_ptr(), S, n, 600, _st()), "embed")
    lg = rng.standard_normal((S, V)).astype(np.float32)
    lg[2, [10, 90000]] = 9.0  # a tie: the first index wins
    lg[4, 777] = np.nan
    tl = _bf16(ON.bf16_round(lg))
    scratch = torch.zeros(-(-L.bp_decode_argmax_rows_scratch_bytes(S) // 4), dtype=torch.int32, device=DEV)
    tok = torch.full((S,), -1, dtype=torch.int64, device=DEV)
    for _ in range(2):  # the counters are left at zero for the next call
        _lib.check(L.bp_decode_argmax_rows(tl.data_ptr(), V, S, tok.data_ptr(), scratch.data_ptr(), _st()), "argmax")
        torch.cuda.synchronize()
        want = [int(np.argmax(ON.bf16_round(row))) for row in lg]
        want[4] = 777
        assert tok.tolist() == want
        assert int(scratch.view(S, -1)[:, -1].abs().sum()) == 0
    torch.cuda.synchronize()
    assert torch.equal(ra.view(torch.int16), rb.view(torch.int16))
    assert torch.equal(sa.view(torch.int16), sb.view(torch.int16))
    assert torch.equal(sc.view(torch.int16), sd.view(torch.int16))
    assert torch.equal(ea, table[ids])


def test_verify_next_accepts_the_matching_prefix_and_advances():
    L = _lib.lib()
    smax = 9
    for s, drafts, toks, want_len in ((1, [], [7], 0), (4, [5, 6, 9], [5, 6, 8, 2], 2), (4, [5, 6, 8], [5, 6, 8, 2], 3),
                                      (9, [1] * 8, [2] + [1] * 8, 0), (3, [4, 4], [4, 4, 4], 2)):
        ids = torch.tensor([3] + drafts + [0] * (smax - s), dtype=torch.int64, device=DEV)
        tok = torch.tensor(toks, dtype=torch.int64, device=DEV)
        out = torch.full((smax + 1,), -5, dtype=torch.int64, device=DEV)
        pos = torch.tensor([100], dtype=torch.int64, device=DEV)
        _lib.check(L.bp_draft_verify_next(ids.data_ptr(), tok.data_ptr(), out.data_ptr(), pos.data_ptr(), s, smax,
                                          _st()), "verify_next")
        torch.cuda.synchronize()
        assert OD.accepted_length([3] + drafts, toks, s - 1) == want_len
        assert int(out[smax]) == want_len and out[:s].tolist() == toks
        assert int(ids[0]) == toks[want_len] and ids[1:s].tolist() == drafts
        assert int(pos) == 100 + want_len + 1


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_verify_rows_match_the_oracle(kind):
    """A verify pass of s rows, teacher-forced after a 5-token prompt: row r's logits against the oracle's decode
    step at that position (within the decode gate), for s = 1 .. 9, and the round's end (accepted length, next
    token and position) against the host's reading of the same row tokens."""
    dec, W, oc = _small_decoder(kind)
    prompt = [3, 17, 99, 250, 7]
    cont = [11, 400, 2, 2, 37, 8, 501, 64, 9]
    kc, vc = OO.new_cache(oc)
    want = []
    for p, t in enumerate(prompt + cont):
        lg = OO.decode_step(W, oc, kc, vc, t, p)
        if p >= len(prompt):
            want.append(lg)
    dec.verify_buffers(9)
    for s in range(1, 10):
        dec.pos.zero_()
        for t in prompt:
            dec.tok.fill_(t)
            dec.step()
        dec.v_ids[:s].copy_(torch.tensor(cont[:s]))
        dec.v_pos.fill_(len(prompt))
        dec.verify(s)
        torch.cuda.synchronize()
        errs = [ON.normwise_error(_np(dec.vlogits[r]), want[r]) for r in range(s)]
        assert max(errs) < GATE, (s, errs)
        toks = dec.v_out[:s].tolist()
        n = OD.accepted_length(cont[:s], toks, s - 1)
        assert int(dec.v_out[dec.smax]) == n and int(dec.v_pos) == len(prompt) + n + 1
        assert int(dec.v_ids[0]) == toks[n]


def _greedy_reference(dec, prompt, n):
    graph = OG.make_generate_graph(dec)
    return graph(prompt, max_new_tokens=n)


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_draft_loop_reproduces_the_graph_loop_olmo2_1b(kind):
    cfg = OG.OLMO2_1B
    print(f"\n[draft] 1B {kind}", flush=True)
    dec = OG.OlmoDecoder(cfg, OG.random_weights(cfg, DEV, seed=4), kind)
    prompt = torch.tensor([[11, 2027, 5, 99999, 42, 3, 3, 1000]])
    n = 40
    ref = _greedy_reference(dec, prompt, n)
    truth = {tuple(prompt[0].tolist()): ref[0, prompt.shape[1]:].tolist()}
    # no drafts: every round is one decode step
    none, _ = OD.make_generate_draft(dec, {"kind": "none", "ks": (0,)})
    assert torch.equal(none(prompt, max_new_tokens=n).cpu(), ref.cpu())
    # the oracle drafter at 2..4 rows per round: every kernel of a row is the one-token step's, bit for bit
    stats = OD.Stats()
    small, _ = OD.make_generate_draft(dec, {"kind": "oracle", "ks": (0, 1, 2, 3), "k_max": 3, "truth": truth}, stats)
    assert torch.equal(small(prompt, max_new_tokens=n).cpu(), ref.cpu())
    assert stats.emitted == n - 1 and stats.rounds <= -(-(n - 1) // 4) + 1, stats.dump()
    # up to 9 and up to 16 rows per round: the same tokens, with no tolerance
    for k_max in (8, 15):
        stats = OD.Stats()
        ks = (0, 1, 2, 4, 6, 8) if k_max == 8 else (0, 1, 3, 7, 11, 15)
        wide, _ = OD.make_generate_draft(dec, {"kind": "oracle", "truth": truth, "ks": ks, "k_max": k_max}, stats)
        out = wide(prompt, max_new_tokens=n)
        assert stats.by_k.get(k_max, 0) >= 1, stats.dump()
        assert out[0, prompt.shape[1]:].tolist() == ref[0, prompt.shape[1]:].tolist(), k_max
    del dec
    torch.cuda.empty_cache()


def test_draft_loop_contract():
    dec, _, _ = _small_decoder("bf16")
    gen, st = OD.make_generate_draft(dec, {"kind": "none"})
    assert st["smax"] == 9
    with pytest.raises(OG.OptimizeError):
        gen(torch.tensor([[1, 2], [3, 4]]), max_new_tokens=3)
    with pytest.raises(OG.OptimizeError):
        gen(torch.tensor([[1, 2]]), max_new_tokens=SMALL.max_len)
    with pytest.raises(OG.OptimizeError):
        OD.make_generate_draft(dec, {"kind": "ngram"})
    oracle, _ = OD.make_generate_draft(dec, {"kind": "oracle", "truth": {}})
    with pytest.raises(OG.OptimizeError):
        oracle(torch.tensor([[1, 2]]), max_new_tokens=4)
    out = gen(torch.tensor([[1, 2, 3]]), max_new_tokens=5, eos_token_id=-1)
    assert out.shape == (1, 8)
