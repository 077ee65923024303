"""The OLMo-2 decode loop on the GPU (byteprof_amd/optim/olmo.py, csrc/decode.hip) against the CPU oracle
(oracle/olmo.py, itself pinned against transformers' Olmo2ForCausalLM in tests/test_oracle_olmo.py).

  - each decode kernel on random inputs against the oracle's function: RMSNorm (+ residual), q/k norm + RoPE +
    cache write (and nothing else written), the attention, SwiGLU, the argmax (ties, NaN) and position update;
  - whole decode steps on a small model, teacher-forced: logits within the decode gate of the oracle, bf16 and int8;
  - the graph loop against the eager loop: the same tokens, bit for bit, over repeated generate calls (graph
    replays with eager work between them), at the small shape and at the OLMo-2-1B shape;
  - the generate() contract of the reference (batch 1 only, the static cache bound, EOS stops the loop).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from byteprof_amd import _lib
from byteprof_amd.optim import olmo as OG
from byteprof_amd.optim.skinny import skinny_mm
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import numerics as ON
from oracle import olmo as OO
from oracle import skinny as OS

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL = OG.OlmoConfig(hidden=256, ffn=512, layers=2, heads=4, vocab=512, max_len=64)
GATE = 2e-2  # max |d| / max |logits|, the gate of tests/test_oracle_olmo.py


def _np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(ON.bf16_round(a))).to(DEV).to(torch.bfloat16)


def _ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 values."""
    ia = ON.bf16_bits(a).astype(np.int32)
    ib = ON.bf16_bits(b).astype(np.int32)
    ia = np.where(ia & 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib & 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)


def _ocfg(cfg: OG.OlmoConfig) -> OO.Config:
    return OO.Config(hidden=cfg.hidden, ffn=cfg.ffn, layers=cfg.layers, heads=cfg.heads, vocab=cfg.vocab,
                     rope_theta=cfg.rope_theta, eps=cfg.eps, max_len=cfg.max_len)


def test_norm_residual_matches_the_oracle():
    rng = np.random.default_rng(0)
    L = _lib.lib()
    for n in (8, 256, 1004, 2048, 3000, 8192, 10000, 16384):  # n % 8 != 0 (1004) takes the scalar kernel
        print(f"\n[olmo] norm n={n}", flush=True)
        x, w, r = (ON.bf16_round(rng.standard_normal(n).astype(np.float32) * s) for s in (3.0, 1.0, 2.0))
        tx, tw, tr = _bf16(x), _bf16(w), _bf16(r)
        out = torch.empty_like(tx)
        st = _lib.stream_ptr(tx.device)
        _lib.check(L.bp_decode_norm_residual(tx.data_ptr(), tw.data_ptr(), None, out.data_ptr(), n, 1e-6, st), "n")
        assert _ulps(_np(out), OO.rmsnorm(x, w, 1e-6)).max() <= 1
        _lib.check(L.bp_decode_norm_residual(tx.data_ptr(), tw.data_ptr(), tr.data_ptr(), tr.data_ptr(), n, 1e-6,
                                             st), "n")  # in place on the residual
        assert _ulps(_np(tr), ON.bf16_round(r + OO.rmsnorm(x, w, 1e-6))).max() <= 1


@pytest.mark.parametrize("with_residual", [True, False])
def test_norm_residual_vector_and_scalar_kernels_agree_bit_for_bit(with_residual):
    """Rows of n % 8 == 0 elements at 16-byte aligned addresses take the vector kernel, other rows the scalar one:
    the same arithmetic in the same order, so the same bits (9 rows of 2048, in place on the residual; the scalar
    kernel reached by offsetting every operand by one element)."""
    L = _lib.lib()
    rng = np.random.default_rng(3)
    S, n = 9, 2048
    x = _bf16(ON.bf16_round(rng.standard_normal((S, n)).astype(np.float32) * 2)).reshape(-1)
    w = _bf16(ON.bf16_round(1 + 0.1 * rng.standard_normal(n).astype(np.float32)))
    r = _bf16(ON.bf16_round(rng.standard_normal((S, n)).astype(np.float32))).reshape(-1)
    outs = []
    for off in (0, 1):
        bufs = [torch.zeros(t.numel() + 8, dtype=torch.bfloat16, device=DEV) for t in (x, w, r)]
        for b, t in zip(bufs, (x, w, r)):
            b[off:off + t.numel()] = t
        bx, bw, br = (b[off:] for b in bufs)
        if with_residual:
            dst, res = br, br.data_ptr()
        else:
            dst, res = torch.zeros_like(br), None
        _lib.check(L.bp_decode_norm_residual_rows(bx.data_ptr(), bw.data_ptr(), res, dst.data_ptr(), n, 1e-6, S,
                                                  _lib.stream_ptr(x.device)), "rows")
        outs.append(dst[:S * n].clone())
    assert torch.equal(outs[0], outs[1])
    ref = np.stack([OO.rmsnorm(row, _np(w), 1e-6) for row in _np(x).reshape(S, n)])
    if with_residual:
        ref = ON.bf16_round(_np(r).reshape(S, n) + ref)
    assert _ulps(_np(outs[0]).reshape(S, n), ref).max() <= 1


@pytest.mark.parametrize("pos", [0, 5, 63])
def test_qk_rope_cache_matches_the_oracle_and_writes_one_cache_row(pos):
    cfg = SMALL
    oc = _ocfg(cfg)
    H, D = cfg.hidden, cfg.head_dim
    rng = np.random.default_rng(pos)
    qkv = ON.bf16_round(rng.standard_normal(3 * H).astype(np.float32))
    qw, kw = (ON.bf16_round(1 + 0.1 * rng.standard_normal(H).astype(np.float32)) for _ in range(2))
    dec_inv = (1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float) / D))).to(DEV)
    np.testing.assert_array_equal(dec_inv.cpu().numpy(), OO.inv_freq(oc))
    kc = torch.full((cfg.heads, cfg.max_len, D), 7.0, dtype=torch.bfloat16, device=DEV)
    vc = torch.full_like(kc, 7.0)
    q_out = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    t_qkv, t_qw, t_kw = _bf16(qkv), _bf16(qw), _bf16(kw)
    _lib.check(_lib.lib().bp_decode_qk_rope_cache(
        t_qkv.data_ptr(), t_qw.data_ptr(), t_kw.data_ptr(), dec_inv.data_ptr(), p.data_ptr(), q_out.data_ptr(),
        kc.data_ptr(), vc.data_ptr(), cfg.heads, D, cfg.max_len, cfg.eps, _lib.stream_ptr(kc.device)), "rope")
    want_q = OO.rope(OO.rmsnorm(qkv[:H], qw, cfg.eps).reshape(cfg.heads, D), pos, oc).reshape(-1)
    want_k = OO.rope(OO.rmsnorm(qkv[H:2 * H], kw, cfg.eps).reshape(cfg.heads, D), pos, oc)
    assert _ulps(_np(q_out), want_q).max() <= 1
    kcn, vcn = _np(kc), _np(vc)
    assert _ulps(kcn[:, pos], want_k).max() <= 1
    np.testing.assert_array_equal(vcn[:, pos], qkv[2 * H:].reshape(cfg.heads, D))
    others = np.ones(cfg.max_len, bool)
    others[pos] = False
    assert (kcn[:, others] == 7.0).all() and (vcn[:, others] == 7.0).all()


# Head dims at both ends of the kernels' range (one to 32 lanes per cache row), and positions that take several row
# batches (up to the longest cache, 4096).
ATTN_CFGS = {"d64": SMALL,
             "d256": OG.OlmoConfig(hidden=512, ffn=512, layers=1, heads=2, vocab=512, max_len=300),
             "d8": OG.OlmoConfig(hidden=64, ffn=512, layers=1, heads=8, vocab=512, max_len=600),
             "d128": OG.OlmoConfig(hidden=512, ffn=512, layers=1, heads=4, vocab=512, max_len=4096)}


@pytest.mark.parametrize("shape,pos", [("d64", 0), ("d64", 1), ("d64", 37), ("d64", 63), ("d256", 299),
                                       ("d8", 599), ("d128", 130), ("d128", 4095)])
def test_attention_matches_the_oracle(shape, pos):
    cfg = ATTN_CFGS[shape]
    oc = _ocfg(cfg)
    D = cfg.head_dim
    rng = np.random.default_rng(100 + pos)
    kc = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    vc = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    q = ON.bf16_round(rng.standard_normal((cfg.heads, D)).astype(np.float32) * 2.0)
    out = torch.empty(cfg.hidden, dtype=torch.bfloat16, device=DEV)
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    tq, tk, tv = _bf16(q), _bf16(kc), _bf16(vc)
    _lib.check(_lib.lib().bp_decode_attention(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), p.data_ptr(),
                                              out.data_ptr(), cfg.heads, D, cfg.max_len, D ** -0.5,
                                              _lib.stream_ptr(out.device)), "attention")
    want = OO.attention(q, kc, vc, pos, oc)
    got = _np(out)
    assert ON.normwise_error(got, want) < 1e-2
    if pos == 0:
        np.testing.assert_array_equal(got, vc[:, 0].reshape(-1))  # one position: the softmax is exactly 1


@pytest.mark.parametrize("shape,pos", [("d64", 0), ("d64", 9), ("d64", 63), ("d256", 299), ("d8", 599),
                                       ("d128", 4095)])
def test_fused_rope_attention_matches_the_oracle(shape, pos):
    """The decode loop's launch: q / k norm + RoPE + cache write + attention for every head at once."""
    cfg = ATTN_CFGS[shape]
    oc = _ocfg(cfg)
    H, D = cfg.hidden, cfg.head_dim
    rng = np.random.default_rng(200 + pos)
    qkv = ON.bf16_round(rng.standard_normal(3 * H).astype(np.float32))
    qw, kw = (ON.bf16_round(1 + 0.1 * rng.standard_normal(H).astype(np.float32)) for _ in range(2))
    kc = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    vc = ON.bf16_round(rng.standard_normal((cfg.heads, cfg.max_len, D)).astype(np.float32))
    tkc, tvc = _bf16(kc), _bf16(vc)
    out = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    inv = torch.from_numpy(OO.inv_freq(oc)).to(DEV)
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    t_qkv, t_qw, t_kw = _bf16(qkv), _bf16(qw), _bf16(kw)
    _lib.check(_lib.lib().bp_decode_rope_attention(
        t_qkv.data_ptr(), t_qw.data_ptr(), t_kw.data_ptr(), inv.data_ptr(), p.data_ptr(), tkc.data_ptr(),
        tvc.data_ptr(), out.data_ptr(), cfg.heads, D, cfg.max_len, cfg.eps, D ** -0.5,
        _lib.stream_ptr(out.device)), "rope_attention")
    q = OO.rope(OO.rmsnorm(qkv[:H], qw, cfg.eps).reshape(cfg.heads, D), pos, oc)
    k = OO.rope(OO.rmsnorm(qkv[H:2 * H], kw, cfg.eps).reshape(cfg.heads, D), pos, oc)
    kc[:, pos], vc[:, pos] = k, qkv[2 * H:].reshape(cfg.heads, D)
    kcn, vcn = _np(tkc), _np(tvc)
    assert _ulps(kcn[:, pos], k).max() <= 1
    np.testing.assert_array_equal(vcn[:, pos], vc[:, pos])
    others = np.ones(cfg.max_len, bool)
    others[pos] = False
    np.testing.assert_array_equal(kcn[:, others], kc[:, others])
    assert ON.normwise_error(_np(out), OO.attention(q, kc, vc, pos, oc)) < 1e-2


@pytest.mark.parametrize("plan", [(1, 4, 0), (2, 2, 0), (4, 8, 0), (1, 4, 1), (2, 2, 1)])
@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_gate_up_silu_equals_the_two_launch_path(kind, plan):
    """The gate|up projection with the SiLU epilogue (bp_skinny_mf_silu) against bp_skinny_mf on the same
    interleaved weight (same plan, split 1) followed by silu_mul on the de-interleaved halves: equal bit for bit;
    within one bf16 step of the oracle. F = 3000 leaves a partial last block."""
    L = _lib.lib()
    F, H = 3000, 2048
    rb, waves, xs = plan
    rng = np.random.default_rng(7 + waves)
    x = _bf16(ON.bf16_round(rng.standard_normal(H).astype(np.float32)))[None]
    w = _bf16(ON.bf16_round(rng.standard_normal((2 * F, H)).astype(np.float32) * 0.05))
    if kind == "bf16":
        args, sc, sdt = (w,), None, 0
    else:
        args = quantize_rowwise_int8(w, torch.float16)
        sc, sdt = args[1].data_ptr(), _lib.TORCH_DT[torch.float16]
    kc = 0 if kind == "bf16" else 1
    out = torch.empty(1, F, dtype=torch.bfloat16, device=DEV)
    st = _lib.stream_ptr(out.device)
    _lib.check(L.bp_skinny_mf_silu(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, out.data_ptr(), 1, F, H, rb, waves,
                                   xs, st), "mf_silu")
    y = torch.empty(1, 2 * F, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_skinny_mf(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, y.data_ptr(), 1, 2 * F, H, rb, waves, 1,
                              xs, None, 0, st), "mf")
    y = y[0]
    gu = torch.cat([y[0::2], y[1::2]]).contiguous()
    ref = torch.empty(F, dtype=torch.bfloat16, device=DEV)
    _lib.check(L.bp_decode_silu_mul(gu.data_ptr(), ref.data_ptr(), F, st), "silu_mul")
    torch.cuda.synchronize()
    assert torch.equal(out[0].view(torch.int16), ref.view(torch.int16))
    g, u = _np(y[0::2]), _np(y[1::2])
    assert _ulps(_np(out[0]), OO.silu_mul(g, u)).max() <= 1
    bad = torch.empty(1, F, dtype=torch.bfloat16, device=DEV)
    assert L.bp_skinny_mf_silu(kc, x.data_ptr(), args[0].data_ptr(), sc, sdt, bad.data_ptr(), 17, F, H, rb, waves, 0,
                               st) == -2  # the epilogue takes at most 16 rows
    assert L.bp_skinny_mf_silu(1, x.data_ptr(), args[0].data_ptr(), None, 1, bad.data_ptr(), 1, F, H, rb, waves, 0,
                               st) == -1  # int8 without a scale


def test_silu_mul_matches_the_oracle():
    rng = np.random.default_rng(3)
    F = 5000
    gu = ON.bf16_round(rng.standard_normal(2 * F).astype(np.float32) * 4.0)
    out = torch.empty(F, dtype=torch.bfloat16, device=DEV)
    t = _bf16(gu)
    _lib.check(_lib.lib().bp_decode_silu_mul(t.data_ptr(), out.data_ptr(), F, _lib.stream_ptr(out.device)), "silu")
    assert _ulps(_np(out), OO.silu_mul(gu[:F], gu[F:])).max() <= 1


def test_argmax_next_takes_the_first_maximum_and_advances_the_position():
    L = _lib.lib()
    st = _lib.stream_ptr(torch.device(DEV))
    scratch = torch.zeros(-(-L.bp_decode_argmax_scratch_bytes() // 4), dtype=torch.int32, device=DEV)
    for V, setup, want in ((100352, {5: 3.0, 70000: 3.0}, 5), (1000, {999: 1.0}, 999), (7, {}, 0),
                           (4096, {10: 2.0, 3000: float("nan")}, 3000)):
        lg = torch.zeros(V, dtype=torch.bfloat16, device=DEV) - 1.0
        for i, v in setup.items():
            lg[i] = v
        tok = torch.tensor([-1], dtype=torch.int64, device=DEV)
        pos = torch.tensor([41], dtype=torch.int64, device=DEV)
        _lib.check(L.bp_decode_argmax_next(lg.data_ptr(), V, tok.data_ptr(), pos.data_ptr(), scratch.data_ptr(), st),
                   "argmax")
        assert int(tok) == want and int(pos) == 42
        assert int(scratch[-1]) == 0  # the ticket counter is back at zero for the next call



@pytest.mark.parametrize("offset", [0, 1])
def test_argmax_next_matches_numpy_on_vector_and_tail_elements(offset):
    """16-byte reads plus the one-at-a-time tail (V not a multiple of 8), and an unaligned buffer (offset 1: every
    element one at a time): the first index of the maximum, NaN counted as largest, -inf everywhere -> 0."""
    L = _lib.lib()
    st = _lib.stream_ptr(torch.device(DEV))
    scratch = torch.zeros(-(-L.bp_decode_argmax_scratch_bytes() // 4), dtype=torch.int32, device=DEV)
    rng = np.random.default_rng(5)
    V = 100351
    cases = [rng.standard_normal(V).astype(np.float32)]
    tie = np.full(V, -2.0, np.float32)
    tie[[3, V - 1]] = 4.0  # a vector element and a tail element tie: the first wins
    cases.append(tie)
    tail = np.full(V, -2.0, np.float32)
    tail[V - 2] = 1.0  # the maximum only in the tail
    cases.append(tail)
    nan = rng.standard_normal(V).astype(np.float32)
    nan[[777, V - 3]] = np.nan
    cases.append(nan)
    cases.append(np.full(V, -np.inf, np.float32))
    for c in cases:
        c = ON.bf16_round(c)
        buf = torch.zeros(V + 8, dtype=torch.bfloat16, device=DEV)
        lg = buf[offset:offset + V]
        lg.copy_(_bf16(c))
        tok = torch.tensor([-1], dtype=torch.int64, device=DEV)
        pos = torch.tensor([0], dtype=torch.int64, device=DEV)
        _lib.check(L.bp_decode_argmax_next(lg.data_ptr(), V, tok.data_ptr(), pos.data_ptr(), scratch.data_ptr(), st),
                   "argmax")
        want = int(np.argmax(c)) if not np.isnan(c).any() else int(np.flatnonzero(np.isnan(c))[0])
        assert int(tok) == want and int(pos) == 1
        assert int(scratch[-1]) == 0


def _deq(args: tuple) -> np.ndarray:
    """q * scale, exact in float32 (8-bit q times an fp16 scale)."""
    q, scale = args
    return q.float().cpu().numpy() * scale.float().cpu().numpy()[:, None]


# a second small shape: hidden a multiple of the 128-byte segment of both kinds (vector loads everywhere)
FUSED_SMALL = OG.OlmoConfig(hidden=1024, ffn=1024, layers=2, heads=8, vocab=512, max_len=64)


def _small_decoder(kind: str, seed: int = 1, cfg: OG.OlmoConfig = SMALL):
    oc = _ocfg(cfg)
    W = OO.random_weights(oc, seed=seed, std=2.0 / np.sqrt(cfg.hidden))
    dec = OG.OlmoDecoder(cfg, {k: _bf16(v) for k, v in W.items()}, kind)
    if kind != "bf16":  # the oracle runs on the weights the kernels see: q * scale, or (code - zero) * scale
        deq = _deq if kind == "int8" else _deq4
        for i, lw in enumerate(dec.layers):
            p = f"l{i}."
            qkv = deq(lw["qkv"])
            H = cfg.hidden
            W[p + "q"], W[p + "k"], W[p + "v"] = qkv[:H], qkv[H:2 * H], qkv[2 * H:]
            gu = deq(lw["gate_up"])
            W[p + "gate"], W[p + "up"] = gu[0::2], gu[1::2]
            W[p + "o"] = deq(lw["o"])
            W[p + "down"] = deq(lw["down"])
        W["lm_head"] = deq(dec.lm_head)
    return dec, W, oc


def _deq4(args) -> np.ndarray:
    """(code - zero) * scale of int4 group-128 weights, exact in float32 (a 4-bit code, an fp16 zero and a bf16
    scale)."""
    packed, scale, zero = args
    return OS.dequantize_int4(packed.cpu().numpy(), scale.float().cpu().numpy(),
                              zero.float().cpu().numpy()).astype(np.float32)


@pytest.mark.parametrize("shape", ["small", "fused"])
@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_decode_steps_match_the_oracle(kind, shape):
    dec, W, oc = _small_decoder(kind, cfg=SMALL if shape == "small" else FUSED_SMALL)
    prompt = [3, 17, 99, 250, 7]
    toks, logits = OO.greedy(W, oc, prompt, 10)
    feed = prompt + toks[:-1]
    dec.pos.zero_()
    errs = []
    for i, t in enumerate(feed):
        dec.tok.fill_(t)
        dec.step()
        if i >= len(prompt) - 1:
            want = logits[i - len(prompt) + 1]
            got = _np(dec.logits[0])
            errs.append(ON.normwise_error(got, want))
            top2 = np.sort(want)[-2:]
            if top2[1] - top2[0] > 2 * errs[-1] * np.abs(want).max():
                assert int(dec.tok) == int(np.argmax(want)), i
    assert int(dec.pos) == len(feed)
    assert max(errs) < GATE, errs


def test_graph_loop_equals_the_eager_loop_small():
    dec, W, oc = _small_decoder("bf16", seed=2)
    eager = OG.make_generate(dec)
    graph = OG.make_generate_graph(dec)
    for prompt in ([1, 2, 3], [400, 9, 9, 9, 17, 250], [5]):
        inp = torch.tensor([prompt])
        a = eager(inp, max_new_tokens=20)
        for _ in range(2):  # the captured graph is reused; eager work runs between the replays
            b = graph(inp, max_new_tokens=20)
            assert torch.equal(a.cpu(), b.cpu()), (prompt, a, b)
        assert a.shape == (1, len(prompt) + 20)
        toks, _ = OO.greedy(W, oc, prompt, 20)
        assert a[0, len(prompt)].item() == toks[0]


def test_generate_contract():
    dec, _, _ = _small_decoder("bf16", seed=3)
    gen = OG.make_generate_graph(dec)
    with pytest.raises(OG.OptimizeError):
        gen(torch.tensor([[1, 2], [3, 4]]), max_new_tokens=4)
    with pytest.raises(OG.OptimizeError):
        gen(torch.tensor([[1, 2]]), max_new_tokens=SMALL.max_len)
    with pytest.raises(OG.OptimizeError):
        gen(torch.tensor([[1, 2]]), max_new_tokens=4, do_sample=True)
    with pytest.raises(OG.OptimizeError):
        gen(torch.tensor([[1, SMALL.vocab]]), max_new_tokens=4)
    full = gen(torch.tensor([[7, 8, 9]]), max_new_tokens=12)
    eager = OG.make_generate(dec)
    # an end-of-sequence id at every place of the two-step groups (the first new token comes from the prompt's last
    # step, then pairs), and runs of every length: the same tokens as the run to 12, cut after the first EOS
    for k in range(6):
        eos = int(full[0, 3 + k])
        first = [int(t) for t in full[0, 3:]].index(eos)
        for g in (gen, eager):
            out = g(torch.tensor([[7, 8, 9]]), max_new_tokens=12, eos_token_id=eos)
            assert torch.equal(out.cpu(), full[:, :3 + first + 1].cpu()), (k, g is gen)
    for n in range(1, 7):
        assert torch.equal(gen(torch.tensor([[7, 8, 9]]), max_new_tokens=n).cpu(), full[:, :3 + n].cpu()), n


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_graph_loop_equals_the_eager_loop_olmo2_1b(kind):
    cfg = OG.OLMO2_1B
    print(f"\n[olmo] 1B {kind}", flush=True)
    dec = OG.OlmoDecoder(cfg, OG.random_weights(cfg, DEV, seed=4), kind)
    prompt = torch.tensor([[11, 2027, 5, 99999, 42, 3, 3, 1000]])
    a = OG.make_generate(dec)(prompt, max_new_tokens=24)
    graph = OG.make_generate_graph(dec)
    for _ in range(2):
        b = graph(prompt, max_new_tokens=24)
        assert torch.equal(a.cpu(), b.cpu())
    assert len(set(a[0, 8:].tolist())) > 1
    del dec
    torch.cuda.empty_cache()


def test_int4_decoder_launch_counts():
    """The int4 decoder: the sublayer norms inside the next linears (bp_skinny_int4_pro) where every plan keeps whole
    rows, else separate norm launches with the SiLU product in the gate|up launch where it keeps whole rows; both
    counted by launches_per_step."""
    dec, _, _ = _small_decoder("int4")
    cfg = SMALL
    H, F = cfg.hidden, cfg.ffn
    whole = all(dec._plan(n, H, 1)[2] == 1 for n in (3 * H, 2 * F, cfg.vocab))
    assert dec.fuse_norms == whole
    if whole:
        assert dec.launches_per_step == 3 + (5 + sum(int(dec._plan(n, k, 1)[2] > 1) for n, k in
                                                     ((H, H), (H, F)))) * cfg.layers
    dec.fuse_norms = False
    per_layer = 7 + sum(int(dec._plan(n, k, 1)[2] > 1) for n, k in
                        ((3 * cfg.hidden, cfg.hidden), (cfg.hidden, cfg.hidden), (cfg.hidden, cfg.ffn))) + \
        2 * int(dec._plan(2 * cfg.ffn, cfg.hidden, 1)[2] > 1)
    assert dec.launches_per_step == 4 + per_layer * cfg.layers + int(dec._plan(cfg.vocab, cfg.hidden, 1)[2] > 1)


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_fused_norm_step_equals_the_separate_norm_step(kind):
    """The step with the sublayer norms inside the next linears (83 launches; the last two norms inside the LM
    head's) gives the logits and tokens of the step with separate norm launches (116 launches), bit for bit, step
    after step."""
    cfg = OG.OLMO2_1B
    print(f"\n[olmo] fused norms {kind}", flush=True)
    dec = OG.OlmoDecoder(cfg, OG.random_weights(cfg, DEV, seed=4), kind)
    assert dec.fuse_norms and dec.launches_per_step == 83
    runs = {}
    for fused in (True, False):
        dec.fuse_norms = fused
        dec.pos.zero_()
        out = []
        for t in (11, 2027, 5, 99999, 42, 3, 3, 1000):
            dec.tok.fill_(t)
            dec.step()
            out.append((dec.logits.clone(), int(dec.tok)))
        runs[fused] = out
    for (la, ta), (lb, tb) in zip(runs[True], runs[False]):
        assert ta == tb and torch.equal(la, lb)
    del dec
    torch.cuda.empty_cache()
