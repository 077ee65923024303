"""OLMo-2 decode step on the CPU (numpy) — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The checker of the graph-captured decode loop (byteprof_amd/optim/olmo.py). The reference's loop (byteprof/optim/olmo.py
:122-219, make_generate_graph) replays the eager forward of HF transformers' Olmo2ForCausalLM (a third-party
dependency, pinned at transformers==4.57.3 in the reference's requirements.txt; 5.15.0 is the version installed
here); this module restates that forward for one token with a static KV cache, with the bf16 roundings of the
model run in bf16 with the eager attention (transformers models/olmo2/modeling_olmo2.py: Olmo2RMSNorm,
Olmo2RotaryEmbedding, apply_rotary_pos_emb, eager_attention_forward, Olmo2MLP, Olmo2DecoderLayer):

  per layer:  q = q_norm(x Wq^T), k = k_norm(x Wk^T), v = x Wv^T            (each linear rounded to bf16)
              q, k = rope(q, pos), rope(k, pos)                              (fp32 cos / sin, one rounding)
              cache[pos] = k, v
              s = bf16(bf16(q . k_t) * head_dim^-0.5), p = bf16(softmax_fp32(s over t <= pos))
              a = bf16(sum_t p_t v_t);  h = x + post_attn_norm(a Wo^T)
              m = bf16(bf16(silu(h Wg^T)) * (h Wu^T));  x' = h + post_ff_norm(m Wd^T)
  head:       logits = bf16(norm(x) Wlm^T);  next token = argmax (first index of the maximum)

RMSNorm: bf16(w * (x * rsqrt(mean(x^2) + eps))) in fp32; residual sums rounded to bf16. The RoPE is that of the
installed transformers (cos / sin kept in fp32); the reference's pinned 4.57.3 rounds cos / sin to bf16 first, a
difference of at most one bf16 step in q and k.

Pinned by tests/test_oracle_olmo.py against transformers' own Olmo2ForCausalLM (eager attention) on the CPU with
the same weights: the logits of every decode step within max |d| / max |logits| < 2e-2 (measured 0.6-1.1e-2: two
to three bf16 steps of the largest logit) and the same greedy tokens, in float32 and in bfloat16; a RoPE rotating
the wrong way planted here moves that error to ~0.5.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .numerics import bf16_round


@dataclass(frozen=True)
class Config:
    hidden: int
    ffn: int
    layers: int
    heads: int
    vocab: int
    rope_theta: float = 500000.0
    eps: float = 1e-6
    max_len: int = 1024

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """bf16(x . w^T) with the products summed in float64 (the skinny kernels' fp32 sum agrees within rounding)."""
    return bf16_round(x.astype(np.float64) @ w.astype(np.float64).T)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float32)
    var = np.mean(x * x, dtype=np.float32)
    return bf16_round(w.astype(np.float32) * (x * np.float32(1.0 / np.sqrt(np.float32(var + np.float32(eps))))))


def inv_freq(cfg: Config) -> np.ndarray:
    """1 / theta^(2i / head_dim) in float32 (Olmo2RotaryEmbedding.compute_default_rope_parameters): the exponent
    in float32, the power correctly rounded to float32 (through float64, as torch's float32 pow gives it), then
    the float32 reciprocal. Equal to torch's values bit for bit (checked in tests/test_olmo_gpu.py)."""
    d = cfg.head_dim
    e = (np.arange(0, d, 2, dtype=np.float32) / np.float32(d)).astype(np.float32)
    p = (np.float64(cfg.rope_theta) ** e.astype(np.float64)).astype(np.float32)
    return (np.float32(1.0) / p).astype(np.float32)


def rope(x: np.ndarray, pos: int, cfg: Config) -> np.ndarray:
    """x [heads, head_dim] (bf16 values) rotated at position pos: bf16(x cos + rotate_half(x) sin), fp32."""
    f = inv_freq(cfg) * np.float32(pos)
    emb = np.concatenate([f, f]).astype(np.float32)
    cos, sin = np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
    half = cfg.head_dim // 2
    rot = np.concatenate([-x[:, half:], x[:, :half]], axis=1)
    return bf16_round(x.astype(np.float32) * cos + rot.astype(np.float32) * sin)


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos: int, cfg: Config) -> np.ndarray:
    """q [heads, d]; kc, vc [heads, max_len, d]; positions 0..pos. Returns [heads * d] (bf16 values)."""
    out = np.zeros((cfg.heads, cfg.head_dim), np.float32)
    scale = np.float32(cfg.head_dim ** -0.5)
    for h in range(cfg.heads):
        k, v = kc[h, :pos + 1].astype(np.float64), vc[h, :pos + 1].astype(np.float64)
        s = bf16_round(bf16_round(k @ q[h].astype(np.float64)) * scale)
        e = np.exp((s - s.max()).astype(np.float64))
        p = bf16_round((e / e.sum()).astype(np.float32))
        out[h] = bf16_round(p.astype(np.float64) @ v)
    return out.reshape(-1)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = g.astype(np.float32)
    a = bf16_round(g / (np.float32(1.0) + np.exp(-g)))
    return bf16_round(a * u.astype(np.float32))


def new_cache(cfg: Config) -> tuple[np.ndarray, np.ndarray]:
    shape = (cfg.layers, cfg.heads, cfg.max_len, cfg.head_dim)
    return np.zeros(shape, np.float32), np.zeros(shape, np.float32)


def decode_step(W: dict, cfg: Config, kc: np.ndarray, vc: np.ndarray, tok: int, pos: int) -> np.ndarray:
    """Logits (bf16 values as float32) of token `tok` at position `pos`; writes the caches at pos. W holds float32
    arrays: embed [V, H]; per layer l (keys 'l{l}.name'): q, k, v, o [H, H], q_norm, k_norm, post_attn, post_ff
    [H], gate, up [F, H], down [H, F]; norm [H], lm_head [V, H]."""
    x = W["embed"][tok].astype(np.float32)
    H, D = cfg.hidden, cfg.head_dim
    for layer in range(cfg.layers):
        p = f"l{layer}."
        q = rmsnorm(linear(x, W[p + "q"]), W[p + "q_norm"], cfg.eps).reshape(cfg.heads, D)
        k = rmsnorm(linear(x, W[p + "k"]), W[p + "k_norm"], cfg.eps).reshape(cfg.heads, D)
        v = linear(x, W[p + "v"]).reshape(cfg.heads, D)
        q, k = rope(q, pos, cfg), rope(k, pos, cfg)
        kc[layer, :, pos], vc[layer, :, pos] = k, v
        a = attention(q, kc[layer], vc[layer], pos, cfg)
        h = bf16_round(x + rmsnorm(linear(a, W[p + "o"]), W[p + "post_attn"], cfg.eps))
        m = silu_mul(linear(h, W[p + "gate"]), linear(h, W[p + "up"]))
        x = bf16_round(h + rmsnorm(linear(m, W[p + "down"]), W[p + "post_ff"], cfg.eps))
    assert x.shape == (H,)
    return linear(rmsnorm(x, W["norm"], cfg.eps), W["lm_head"])


def greedy(W: dict, cfg: Config, prompt: list[int], new_tokens: int) -> tuple[list[int], list[np.ndarray]]:
    """Greedy decoding token by token (the prompt fed one position at a time): the new tokens and the logits of
    every step from the last prompt position on."""
    kc, vc = new_cache(cfg)
    logits = None
    for pos, t in enumerate(prompt):
        logits = decode_step(W, cfg, kc, vc, t, pos)
    out, all_logits = [], [logits]
    pos = len(prompt)
    for i in range(new_tokens):
        t = int(np.argmax(logits))
        out.append(t)
        if i + 1 == new_tokens:
            break
        logits = decode_step(W, cfg, kc, vc, t, pos)
        all_logits.append(logits)
        pos += 1
    return out, all_logits


def random_weights(cfg: Config, seed: int = 0, std: float = 0.02) -> dict:
    """Seeded synthetic weights (bf16 values): linears ~ N(0, std^2), norm weights ~ 1 + N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    H, F, V = cfg.hidden, cfg.ffn, cfg.vocab

    def lin(n, k):
        return bf16_round(rng.standard_normal((n, k), dtype=np.float32) * np.float32(std))

    def norm(n):
        return bf16_round(1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32))

    W = {"embed": bf16_round(rng.standard_normal((V, H), dtype=np.float32))}
    for layer in range(cfg.layers):
        p = f"l{layer}."
        W[p + "q"], W[p + "k"], W[p + "v"], W[p + "o"] = lin(H, H), lin(H, H), lin(H, H), lin(H, H)
        W[p + "q_norm"], W[p + "k_norm"] = norm(H), norm(H)
        W[p + "post_attn"], W[p + "post_ff"] = norm(H), norm(H)
        W[p + "gate"], W[p + "up"], W[p + "down"] = lin(F, H), lin(F, H), lin(H, F)
    W["norm"] = norm(H)
    W["lm_head"] = lin(V, H)
    return W
