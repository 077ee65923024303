"""Pins oracle/olmo.py (the OLMo-2 decode step) against transformers' own Olmo2ForCausalLM on the CPU.

The reference's decode loop (byteprof/optim/olmo.py:122-219) replays the eager forward of that model; here the
same seeded weights go into both, and every decode step is compared teacher-forced (both fed the oracle's greedy
tokens): logits within max |d| / max |logits| < 2e-2 (measured: 0.6-1.1e-2, two to three bf16 steps of the
largest logit, from intermediate bf16 values that round differently under other summation orders) in float32
and in bfloat16 (eager attention), and the greedy token equal wherever the top two logits are further apart than
the error. A mistake planted in the oracle (RoPE rotating the wrong way, the attention scale off by a factor
head_dim^(1/4), a norm weight dropped) moves the error to 0.3-0.9, far outside the gate (the first is a test
below). Also pinned by hand: RMSNorm of a constant vector, RoPE at position 0 (identity) and its norm
preservation, and the attention over one position (returns v).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import olmo as OO
from oracle import numerics as ON

CFG = OO.Config(hidden=256, ffn=512, layers=2, heads=4, vocab=512, max_len=64)
PROMPT = [3, 17, 99, 250, 7]
GATE = 2e-2


def _hf_model(cfg: OO.Config, W: dict, dtype):
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    hc = tr.Olmo2Config(hidden_size=cfg.hidden, intermediate_size=cfg.ffn, num_hidden_layers=cfg.layers,
                        num_attention_heads=cfg.heads, num_key_value_heads=cfg.heads, vocab_size=cfg.vocab,
                        max_position_embeddings=cfg.max_len, rms_norm_eps=cfg.eps, attention_bias=False,
                        tie_word_embeddings=False, eos_token_id=None, pad_token_id=None, bos_token_id=None,
                        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta})
    hc._attn_implementation = "eager"
    m = tr.Olmo2ForCausalLM(hc).eval()
    sd = {"model.embed_tokens.weight": W["embed"], "model.norm.weight": W["norm"], "lm_head.weight": W["lm_head"]}
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm", "post_attn": "post_attention_layernorm",
             "post_ff": "post_feedforward_layernorm", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
             "down": "mlp.down_proj"}
    for layer in range(cfg.layers):
        for ours, theirs in names.items():
            sd[f"model.layers.{layer}.{theirs}.weight"] = W[f"l{layer}.{ours}"]
    result = m.load_state_dict({k: torch.from_numpy(v.copy()) for k, v in sd.items()}, strict=True)
    assert not result.missing_keys and not result.unexpected_keys
    return m.to(dtype)


def _teacher_forced_errors(m, toks, logits):
    """Per-step max |d| / max |logits| of the HF model fed the oracle's tokens, and whether each clear argmax agrees."""
    torch = pytest.importorskip("torch")
    errs, agree = [], []
    with torch.no_grad():
        out = m(torch.tensor([PROMPT]), use_cache=True)
        pkv = out.past_key_values
        for i, want in enumerate(logits):
            got = out.logits[0, -1].float().numpy()
            errs.append(ON.normwise_error(got, want))
            top2 = np.sort(want)[-2:]
            if (top2[1] - top2[0]) > 2 * errs[-1] * np.abs(want).max():
                agree.append(int(np.argmax(got)) == toks[i])
            if i + 1 < len(logits):
                out = m(torch.tensor([[toks[i]]]), past_key_values=pkv, use_cache=True)
                pkv = out.past_key_values
    return errs, agree


@pytest.mark.parametrize("dtype_name", ["float32", "bfloat16"])
def test_olmo_oracle_matches_transformers(dtype_name):
    torch = pytest.importorskip("torch")
    W = OO.random_weights(CFG, seed=1, std=2.0 / np.sqrt(CFG.hidden))
    toks, logits = OO.greedy(W, CFG, PROMPT, 10)
    errs, agree = _teacher_forced_errors(_hf_model(CFG, W, getattr(torch, dtype_name)), toks, logits)
    assert max(errs) < GATE, errs
    assert agree and all(agree), agree
    assert len(set(toks)) > 3  # the synthetic model does not just repeat one token


def test_a_mistake_planted_in_the_oracle_fails_the_gate(monkeypatch):
    torch = pytest.importorskip("torch")
    W = OO.random_weights(CFG, seed=1, std=2.0 / np.sqrt(CFG.hidden))
    m = _hf_model(CFG, W, torch.float32)
    rope = OO.rope
    monkeypatch.setattr(OO, "rope", lambda x, pos, cfg: rope(x, -pos, cfg))  # rotating the wrong way
    toks, logits = OO.greedy(W, CFG, PROMPT, 6)
    errs, _ = _teacher_forced_errors(m, toks, logits)
    assert max(errs) > 10 * GATE, errs


def test_rmsnorm_of_a_constant_vector():
    x = np.full(64, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    np.testing.assert_array_equal(OO.rmsnorm(x, w, 0.0), ON.bf16_round(w))


def test_rope_at_position_zero_is_the_identity_and_preserves_norms():
    rng = np.random.default_rng(0)
    x = ON.bf16_round(rng.standard_normal((CFG.heads, CFG.head_dim)).astype(np.float32))
    np.testing.assert_array_equal(OO.rope(x, 0, CFG), x)
    y = OO.rope(x, 37, CFG)
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-2)
    # pairs (i, i + d/2) rotate by 37 * inv_freq[i]: the first pair at angle 37 rad
    half = CFG.head_dim // 2
    a = 37.0
    want = x[0, 0] * np.cos(a) - x[0, half] * np.sin(a)
    assert abs(y[0, 0] - want) <= 2 ** -7 * max(abs(want), 1e-3)


def test_attention_over_one_position_returns_v():
    rng = np.random.default_rng(1)
    kc = np.zeros((CFG.heads, CFG.max_len, CFG.head_dim), np.float32)
    vc = np.zeros_like(kc)
    kc[:, 0] = ON.bf16_round(rng.standard_normal((CFG.heads, CFG.head_dim)).astype(np.float32))
    vc[:, 0] = ON.bf16_round(rng.standard_normal((CFG.heads, CFG.head_dim)).astype(np.float32))
    q = ON.bf16_round(rng.standard_normal((CFG.heads, CFG.head_dim)).astype(np.float32))
    np.testing.assert_array_equal(OO.attention(q, kc, vc, 0, CFG), vc[:, 0].reshape(-1))
