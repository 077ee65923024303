"""OLMo-2 decode loop on gfx950: the whole decode step (skinny linears + the decode kernels of csrc/decode.hip, 83
launches for the 16-layer model: each sublayer norm and residual add runs inside the next linear's launch, the
last layer's and the final norm both inside the LM head's) captured
in HIP graphs of two steps, each step's token copied to pinned memory inside the graph; greedy generation replays
them one replay ahead of the host (one event synchronize per two tokens).

Drop-in for the loops of byteprof/optim/olmo.py: `make_generate_graph` (olmo.py:122-219, the manually captured
graph of the eager forward incl. argmax and next-step inputs) and `make_generate` (olmo.py:51-119, the minimal
loop: the same step run eagerly, one read per token). Both return `generate(inputs, max_new_tokens=...)` with the
reference's contract: batch 1 and greedy only (OptimizeError otherwise), the prompt plus the new tokens within the
static cache (MAX_CACHE_LEN), generation stops after an EOS id or max_new_tokens, and the result is the prompt
followed by the new tokens, [1, L + n].

The model is the OLMo-2 architecture with synthetic weights (the checkpoint is not available here): an
`OlmoDecoder` holds the weights of transformers' Olmo2ForCausalLM layout with q|k|v and gate|up fused into one
linear each (one launch instead of three or two; the outputs are the same rows), bf16, int8 (per-row scales) or
int4 (group-128 codes). The gate and up rows are interleaved (row 2n gate n, row 2n + 1 up n) so that one launch
computes the projection and the SiLU product (bp_skinny_mf_silu, bp_skinny_int4_silu). Every linear runs on a
matrix-core kernel whose rows do not depend on how many rows share a launch: a verify pass of s rows computes each
row exactly as the one-token step.
The prompt is fed one position at a time through the same step (the reference prefills with one batched
forward; the cache contents and the first new token are the same up to rounding).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from .. import _lib
from ..quant.hip_int8 import quantize_rowwise_int8
from . import skinny as S

MAX_CACHE_LEN = 1024  # the reference's static cache length (olmo.py:16)
ROPE_ATTENTION_ROWS = 16  # most rows of one fused q/k-norm + RoPE + cache + attention launch
VERIFY_ROWS = 16  # rows of the verify-pass buffers (allocated once per decoder, never reallocated)
PRO_MAX_ROWS = {"bf16": 3, "int8": 1, "int4": 1}  # most rows of a linear launch with the norm as its prologue
INT4_PRO_LDS_BYTES = 64 * 1024  # the int4 kernel's norm prologue: rows, gamma, residual rows, gamma2, (2 M + 2) K bf16
INT4_PRO_MAX_K = INT4_PRO_LDS_BYTES // 8  # widest row it stages at one row
PRO_LDS_BYTES = 80 * 1024  # the launch keeps gamma and the residual rows in LDS while the staged rows and they fit
ARGMAX_ROW_WORDS, ARGMAX_ERROR_WORD = 132, 130  # u32 words of the argmax scratch per row; its error word


class OptimizeError(RuntimeError):
    """A generate() call outside what the loop supports (the reference's byteprof.optim.OptimizeError)."""


@dataclass(frozen=True)
class OlmoConfig:
    hidden: int
    ffn: int
    layers: int
    heads: int
    vocab: int
    rope_theta: float = 500000.0
    eps: float = 1e-6
    max_len: int = MAX_CACHE_LEN

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


# allenai/OLMo-2-0425-1B: 16 layers, hidden 2048, FFN 8192, 16 heads of 128, vocabulary 100352
OLMO2_1B = OlmoConfig(hidden=2048, ffn=8192, layers=16, heads=16, vocab=100352)

LAYER_WEIGHTS = ("q", "k", "v", "o", "q_norm", "k_norm", "post_attn", "gate", "up", "down", "post_ff")


def random_weights(cfg: OlmoConfig, device, seed: int = 0, std: float | None = None) -> dict[str, torch.Tensor]:
    """Seeded synthetic bf16 weights on `device`, keyed like oracle/olmo.py (embed, l{i}.{q,k,v,o,q_norm,k_norm,
    post_attn,gate,up,down,post_ff}, norm, lm_head): linears ~ N(0, std^2) with std = 2 / sqrt(hidden) by default,
    norm weights ~ 1 + N(0, 0.1^2), embeddings ~ N(0, 1)."""
    g = torch.Generator(device=device).manual_seed(seed)
    std = 2.0 / cfg.hidden ** 0.5 if std is None else std
    H, F, V = cfg.hidden, cfg.ffn, cfg.vocab

    def lin(n, k):
        return (torch.randn(n, k, generator=g, device=device) * std).to(torch.bfloat16)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

    W = {"embed": torch.randn(V, H, generator=g, device=device).to(torch.bfloat16)}
    for layer in range(cfg.layers):
        p = f"l{layer}."
        for name in ("q", "k", "v", "o"):
            W[p + name] = lin(H, H)
        for name in ("q_norm", "k_norm", "post_attn", "post_ff"):
            W[p + name] = norm(H)
        W[p + "gate"], W[p + "up"], W[p + "down"] = lin(F, H), lin(F, H), lin(H, F)
    W["norm"] = norm(H)
    W["lm_head"] = lin(V, H)
    return W


class OlmoDecoder:
    """One OLMo-2 decode step on the GPU, reading the token id and the position from device memory (tok, pos) and
    leaving the next token in tok and pos + 1 in pos. kind: 'bf16', 'int8' (every linear quantized per row, fp16
    scales) or 'int4' (group-128 codes with per-group scale and zero, tile-major at the tuned tile rows: the int4_wo
    format of skinny_mm; its steps run the norms as launches of their own, and drafting verify passes take bf16 or
    int8 only); embeddings and norm weights stay bf16."""

    def __init__(self, cfg: OlmoConfig, weights: dict[str, torch.Tensor], kind: str = "bf16"):
        if kind not in ("bf16", "int8", "int4"):
            raise ValueError("kind must be 'bf16', 'int8' or 'int4'")
        if cfg.hidden % cfg.heads or cfg.head_dim % 8 or 256 % cfg.head_dim or cfg.max_len > 4096:
            raise ValueError("head_dim must be a multiple of 8 dividing 256 and max_len at most 4096")
        self.cfg, self.kind = cfg, kind
        dev = weights["embed"].device
        if dev.type != "cuda":
            raise ValueError("the decoder runs on the GPU only")
        self.device = dev
        H, F, V, D = cfg.hidden, cfg.ffn, cfg.vocab, cfg.head_dim

        def lin(w: torch.Tensor) -> tuple:
            w = w.contiguous()
            if kind == "int4":
                return S.quantize_int4(w, S.int4_tile_rows(*w.shape))
            return (w,) if kind == "bf16" else quantize_rowwise_int8(w, torch.float16)

        bf = torch.bfloat16

        def gate_up(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:  # rows interleaved: 2f gate f, 2f + 1 up f
            return torch.stack([g, u], dim=1).reshape(2 * F, H)

        self.embed = weights["embed"].to(bf).contiguous()
        self.norm = weights["norm"].to(bf).contiguous()
        self.lm_head = lin(weights["lm_head"])
        self.layers = []
        for layer in range(cfg.layers):
            p = f"l{layer}."
            self.layers.append({
                "qkv": lin(torch.cat([weights[p + "q"], weights[p + "k"], weights[p + "v"]])),
                "o": lin(weights[p + "o"]),
                "gate_up": lin(gate_up(weights[p + "gate"], weights[p + "up"])),
                "down": lin(weights[p + "down"]),
                **{n: weights[p + n].to(bf).contiguous() for n in ("q_norm", "k_norm", "post_attn", "post_ff")},
            })
        # Olmo2RotaryEmbedding.compute_default_rope_parameters, in float32 on the host
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float) / D))).to(dev)
        self.scale = float(D) ** -0.5
        z = lambda *shape, dtype=bf: torch.zeros(*shape, dtype=dtype, device=dev)  # noqa: E731
        self.tok, self.pos = z(1, dtype=torch.int64), z(1, dtype=torch.int64)
        self.x, self.xn, self.attn, self.o, self.dn = z(1, H), z(1, H), z(1, H), z(1, H), z(1, H)
        self.h = z(1, H)  # the residual stream after the attention half of a layer (fused-norm step)
        # the sublayer norms run inside the next linear's launch when its plan keeps whole rows (split 1); the int4
        # kernel's prologue stages the row, gamma, the residual row and gamma2 in LDS (K <= 8192, bf16 scales)
        self.fuse_norms = all(self._plan(n, H, 1)[2] == 1 for n in (3 * H, 2 * F, V)) and (
            kind != "int4" or (H <= INT4_PRO_MAX_K and self.lm_head[1].dtype == torch.bfloat16))
        self.qkv, self.gu, self.act, self.logits = z(1, 3 * H), z(1, 2 * F), z(1, F), z(1, V)
        # the argmax's partials, counter and error word: zeroed once, the counter left at zero by every launch
        self.argmax_scratch = z(-(-_lib.lib().bp_decode_argmax_scratch_bytes() // 4), dtype=torch.int32)
        self.k_cache = z(cfg.layers, cfg.heads, cfg.max_len, D)
        self.v_cache = z(cfg.layers, cfg.heads, cfg.max_len, D)

    @staticmethod
    def _mm(x: torch.Tensor, args: tuple, out: torch.Tensor) -> None:
        S.skinny_mm(x, *args, out=out)

    def step(self) -> None:
        """Logits of token tok at position pos; then tok <- argmax, pos <- pos + 1 (all on the device)."""
        if self.fuse_norms:
            self._step_fused()
        else:
            self._step_separate()

    def _step_fused(self) -> None:
        """The step with each sublayer norm and residual add inside the next linear's launch (bp_skinny_mf_pro,
        BP_PRO_NORM: the norm kernel's arithmetic, so the tokens are those of the separate-norm step): q|k|v of
        layer l > 0 reads down_{l-1} and writes the residual stream x_l; gate|up reads o and writes h_l = x_l +
        norm(o); the last layer's post-feed-forward norm and the final norm both run inside the LM head's launch.
        x and h alternate, so no launch reads what it writes."""
        cfg, L = self.cfg, _lib.lib()
        H, D = cfg.hidden, cfg.head_dim
        st = _lib.stream_ptr(self.device)
        c = _lib.check
        c(L.bp_decode_embed(self.tok.data_ptr(), self.embed.data_ptr(), self.x.data_ptr(), H, cfg.vocab, st),
          "bp_decode_embed")
        for i, w in enumerate(self.layers):
            kc, vc = self.k_cache[i], self.v_cache[i]
            if i == 0:
                self._mm(self.x, w["qkv"], self.qkv)
            else:
                self._pro_mm(self.dn, w["qkv"], self.qkv, self.layers[i - 1]["post_ff"], self.h, self.x)
            c(L.bp_decode_rope_attention(self.qkv.data_ptr(), w["q_norm"].data_ptr(), w["k_norm"].data_ptr(),
                                         self.inv_freq.data_ptr(), self.pos.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                         self.attn.data_ptr(), cfg.heads, D, cfg.max_len, cfg.eps, self.scale, st),
              "bp_decode_rope_attention")
            self._mm(self.attn, w["o"], self.o)
            self._pro_mm(self.o, w["gate_up"], self.act, w["post_attn"], self.x, self.h, silu=True)
            self._mm(self.act, w["down"], self.dn)
        self._pro_mm(self.dn, self.lm_head, self.logits, self.layers[-1]["post_ff"], self.h, self.x, gamma2=self.norm)
        c(L.bp_decode_argmax_next(self.logits.data_ptr(), cfg.vocab, self.tok.data_ptr(), self.pos.data_ptr(),
                                  self.argmax_scratch.data_ptr(), st), "bp_decode_argmax_next")

    def _pro_mm(self, x: torch.Tensor, args: tuple, out: torch.Tensor, gamma: torch.Tensor,
                residual: torch.Tensor | None, xout: torch.Tensor | None, silu: bool = False,
                gamma2: torch.Tensor | None = None) -> None:
        """out = linear(bf16(residual + bf16(gamma * rmsnorm(x)))) in one launch (with gamma2: linear of the
        gamma2-norm of that); xout receives the normalised rows (the new residual stream)."""
        S.prologue_mm(x, args[0], args[1] if len(args) > 1 else None, out, S.PRO_NORM, gamma=gamma,
                      residual=residual, xout=xout, eps=self.cfg.eps, silu=silu, gamma2=gamma2,
                      zero=args[2] if len(args) > 2 else None)

    def _step_separate(self) -> None:
        """The step with a norm launch after o and after down (plans that split K)."""
        cfg, L = self.cfg, _lib.lib()
        H, D = cfg.hidden, cfg.head_dim
        st = _lib.stream_ptr(self.device)
        c = _lib.check
        c(L.bp_decode_embed(self.tok.data_ptr(), self.embed.data_ptr(), self.x.data_ptr(), H, cfg.vocab, st),
          "bp_decode_embed")
        for i, w in enumerate(self.layers):
            kc, vc = self.k_cache[i], self.v_cache[i]
            self._mm(self.x, w["qkv"], self.qkv)
            c(L.bp_decode_rope_attention(self.qkv.data_ptr(), w["q_norm"].data_ptr(), w["k_norm"].data_ptr(),
                                         self.inv_freq.data_ptr(), self.pos.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                         self.attn.data_ptr(), cfg.heads, D, cfg.max_len, cfg.eps, self.scale, st),
              "bp_decode_rope_attention")
            self._mm(self.attn, w["o"], self.o)
            c(L.bp_decode_norm_residual(self.o.data_ptr(), w["post_attn"].data_ptr(), self.x.data_ptr(),
                                        self.x.data_ptr(), H, cfg.eps, st), "bp_decode_norm_residual")
            self._gate_up_silu(self.x, w["gate_up"], self.act, self.gu, 1)
            self._mm(self.act, w["down"], self.dn)
            c(L.bp_decode_norm_residual(self.dn.data_ptr(), w["post_ff"].data_ptr(), self.x.data_ptr(),
                                        self.x.data_ptr(), H, cfg.eps, st), "bp_decode_norm_residual")
        c(L.bp_decode_norm_residual(self.x.data_ptr(), self.norm.data_ptr(), None, self.xn.data_ptr(), H, cfg.eps,
                                    st), "bp_decode_norm_residual")
        self._mm(self.xn, self.lm_head, self.logits)
        c(L.bp_decode_argmax_next(self.logits.data_ptr(), cfg.vocab, self.tok.data_ptr(), self.pos.data_ptr(),
                                  self.argmax_scratch.data_ptr(), st), "bp_decode_argmax_next")

    def _plan(self, n: int, k: int, rows: int) -> tuple[int, int, int, int]:
        """(weight blocks per workgroup, waves, split, staging) of the skinny launch skinny_mm makes (int4: the tile
        rows' 16-row blocks, waves, split, no staging)."""
        if self.kind == "int4":
            tile = S.int4_tile_rows(n, k)
            waves, split = S.int4_cfg(n, k, tile)
            return tile // 16, waves, min(split, k // 128), 0
        return S._resolve(self.kind, n, k, rows, None)

    def _gate_up_silu(self, x: torch.Tensor, gw: tuple, act: torch.Tensor, gu: torch.Tensor, rows: int) -> None:
        """act[:rows] = bf16(bf16(silu(g)) * u) of the interleaved gate|up projection: one launch with the SiLU
        product as its epilogue when the shape's K order has no split, else skinny_mm + the SiLU kernel (the same
        sums either way)."""
        F, H = self.cfg.ffn, self.cfg.hidden
        rb, waves, split, xs = self._plan(2 * F, H, rows)
        L, st = _lib.lib(), _lib.stream_ptr(self.device)
        if self.kind == "int4" and split == 1 and rows <= 16 and F % 2 == 0:
            packed, scale, zero = gw
            _lib.check(L.bp_skinny_int4_silu(x.data_ptr(), packed.data_ptr(), scale.data_ptr(),
                                             _lib.TORCH_DT[scale.dtype], zero.data_ptr(), act.data_ptr(), rows, F, H,
                                             16 * rb, waves, st), "bp_skinny_int4_silu")
            return
        if split == 1 and rows <= 16 and self.kind != "int4":
            sc, sdt = (gw[1].data_ptr(), _lib.TORCH_DT[gw[1].dtype]) if self.kind == "int8" else (None, 0)
            _lib.check(L.bp_skinny_mf_silu(S._KIND_CODE[self.kind], x.data_ptr(), gw[0].data_ptr(), sc, sdt,
                                           act.data_ptr(), rows, F, H, rb, waves, xs, st), "bp_skinny_mf_silu")
            return
        self._mm(x[:rows], gw, gu[:rows])
        _lib.check(L.bp_decode_silu_mul_rows(gu.data_ptr(), act.data_ptr(), F, rows, 1, st), "bp_decode_silu_mul_rows")

    @property
    def launches_per_step(self) -> int:
        """Kernel launches of one step. Fused norms: embed, 5 per layer (q|k|v, RoPE + attention, o, gate|up,
        down; + 1 per split-K o or down), the LM head with the last two norms, argmax. Separate norms: embed, 7 per
        layer (+1 per split-K linear), final norm, LM head, argmax."""
        H, F, V = self.cfg.hidden, self.cfg.ffn, self.cfg.vocab
        extra = lambda n, k: int(self._plan(n, k, 1)[2] > 1)  # noqa: E731  (the split reduce)
        if self.fuse_norms:
            return 3 + (5 + extra(H, H) + extra(H, F)) * self.cfg.layers
        # gate|up: the SiLU epilogue in the launch, else the product's own launch after a split's reduce
        per_layer = 7 + extra(3 * H, H) + extra(H, H) + extra(H, F) + 2 * extra(2 * F, H)
        return 4 + per_layer * self.cfg.layers + extra(V, H)

    def _down_splitk(self, s: int) -> tuple[int, int, int, int] | None:
        """The down projection's plan at s rows when it is split-K (its partials then feed the norm's launch)."""
        H, F = self.cfg.hidden, self.cfg.ffn
        if self.kind == "int4":  # no partials entry for int4 weights: skinny_mm reduces, a norm launch follows
            return None
        plan = self._plan(H, F, s)
        return plan if plan[2] > 1 and H <= 8192 else None

    def verify_buffers(self, smax: int) -> None:
        """The buffers of verify passes (allocated once, for VERIFY_ROWS rows, and never reallocated, so graphs
        captured by any drafting loop on this decoder keep valid pointers). ids [VERIFY_ROWS] and pos [1] (int64) are
        a round's inputs: ids[0] the last accepted token, ids[1 ..] the drafts, pos the cache position of ids[0];
        out [VERIFY_ROWS + 1] receives the row tokens and, at VERIFY_ROWS (= self.smax), the accepted length."""
        if not 1 <= smax <= VERIFY_ROWS:
            raise ValueError(f"verify passes take 1..{VERIFY_ROWS} rows, asked for {smax}")
        if getattr(self, "smax", 0):
            return
        cfg, dev = self.cfg, self.device
        H, F, V = cfg.hidden, cfg.ffn, cfg.vocab
        n = VERIFY_ROWS
        z = lambda *shape, dtype=torch.bfloat16: torch.zeros(*shape, dtype=dtype, device=dev)  # noqa: E731
        self.smax = n
        self.v_ids, self.v_tok, self.v_out = z(n, dtype=torch.int64), z(n, dtype=torch.int64), \
            z(n + 1, dtype=torch.int64)
        self.v_pos = z(1, dtype=torch.int64)
        self.vx, self.vh, self.vq, self.vattn, self.vo, self.vdn, self.vxn = (z(n, H) for _ in range(7))
        self.vqkv, self.vgu, self.vact, self.vlogits = z(n, 3 * H), z(n, 2 * F), z(n, F), z(n, V)
        self.v_argmax_scratch = z(-(-_lib.lib().bp_decode_argmax_rows_scratch_bytes(n) // 4), dtype=torch.int32)
        split = max(p[2] for p in (self._plan(H, F, r) for r in range(1, n + 1)))
        self.vws = torch.empty(split * n * H, dtype=torch.float32, device=dev)  # the down launch's partials

    def _pro_fits(self, n: int, k: int, rows: int, norms: int = 1) -> bool:
        """Whether the launch of an n x k linear at rows rows takes a norm prologue: a plan that keeps whole rows
        (split 1), the rows x k activations staged in LDS (32 KiB), gamma with the residual rows in LDS beside them
        (one row, or PRO_LDS_BYTES in all: past it the prologue would read them from memory element by element, which
        made 7-row verify rounds 870 -> 1206 us), and at most PRO_MAX_ROWS rows: measured on the OLMo-2-1B shape
        against the one-round-trip norm launch, the prologue wins at 1..3 rows for bf16 (2 / 3-row rounds 731 / 755
        -> 724 / 749 us; 5 rows loses, 791-808 -> 829 us) and at one row only for int8 (2 / 3 rows: 575 / 586-599
        without it, 587-597 / 631-634 with it) and for int4 (2 / 3 / 5 / 7 rows: 601 / 617 / 642 / 681 us without it,
        619 / 654 / 746 / 867 with it); at one row it saves the norm launch of every sublayer."""
        _, _, split, _ = self._plan(n, k, rows)
        if split != 1 or rows > PRO_MAX_ROWS[self.kind]:
            return False
        if self.kind == "int4":  # the int4 kernel's prologue (rows, gamma, residual rows, gamma2 in LDS)
            return (2 * rows + 2) * k * 2 <= INT4_PRO_LDS_BYTES and self.lm_head[1].dtype == torch.bfloat16
        st = S._stage_bytes(self.kind, rows, k, 1)
        return st >= 0 and (rows == 1 or st + 2 * k * (norms + rows) <= PRO_LDS_BYTES)

    def verify(self, s: int) -> None:
        """One verify pass of s = 1 + drafts rows (the reference's captured draft step, olmo_draft.py
        make_generate_draft): ids[:s] at positions pos .. pos + s - 1 through the model with the static cache (the
        rows' k / v written first, row r attending over positions <= pos + r), the argmax of every row, the accepted
        length L (drafts ids[1 + j] equal to the prediction of row j) and the next round's inputs: ids[0] <- the
        token after the accepted prefix, pos += L + 1. Every row is computed as the one-token step at its position
        computes it (the linears' rows do not depend on the row count). Each sublayer norm runs inside the next
        linear's launch where _pro_fits allows (up to 3 bf16 rows / one int8 or int4 row), else as its own launch
        (the same bits either way); the residual stream alternates between vx and vh where a prologue writes it."""
        if not 1 <= s <= getattr(self, "smax", 0):
            raise ValueError(f"s must be in 1..{getattr(self, 'smax', 0)} (verify_buffers)")
        cfg, L = self.cfg, _lib.lib()
        H, F, V = cfg.hidden, cfg.ffn, cfg.vocab
        st = _lib.stream_ptr(self.device)
        c = _lib.check
        c(L.bp_decode_embed_rows(self.v_ids.data_ptr(), self.embed.data_ptr(), self.vx.data_ptr(), s, H, cfg.vocab,
                                 st), "bp_decode_embed_rows")
        res, spare = self.vx, self.vh  # the residual stream [s, H] and the buffer a prologue writes the next one to
        pending = None  # the post-feed-forward norm weight still to apply to vdn (with the residual add)

        def norm_into(src: torch.Tensor, gamma: torch.Tensor) -> None:  # res <- res + norm(src), in place
            c(L.bp_decode_norm_residual_rows(src.data_ptr(), gamma.data_ptr(), res.data_ptr(), res.data_ptr(), H,
                                             cfg.eps, s, st), "bp_decode_norm_residual_rows")

        for i, w in enumerate(self.layers):
            kc, vc = self.k_cache[i], self.v_cache[i]
            if pending is not None and self._pro_fits(3 * H, H, s):
                self._pro_mm(self.vdn[:s], w["qkv"], self.vqkv[:s], pending, res[:s], spare[:s])
                res, spare = spare, res
            else:
                if pending is not None:
                    norm_into(self.vdn, pending)
                self._mm(res[:s], w["qkv"], self.vqkv[:s])
            pending = None
            if s <= ROPE_ATTENTION_ROWS:  # one fused launch (equal bit for bit to the two below)
                c(L.bp_decode_rope_attention_rows(self.vqkv.data_ptr(), w["q_norm"].data_ptr(),
                                                  w["k_norm"].data_ptr(), self.inv_freq.data_ptr(),
                                                  self.v_pos.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                                  self.vattn.data_ptr(), cfg.heads, cfg.head_dim, s, cfg.max_len,
                                                  cfg.eps, self.scale, st), "bp_decode_rope_attention_rows")
            else:
                c(L.bp_decode_qk_rope_cache_rows(self.vqkv.data_ptr(), w["q_norm"].data_ptr(),
                                                 w["k_norm"].data_ptr(), self.inv_freq.data_ptr(),
                                                 self.v_pos.data_ptr(), self.vq.data_ptr(), kc.data_ptr(),
                                                 vc.data_ptr(), cfg.heads, cfg.head_dim, cfg.max_len, cfg.eps, s, st),
                  "bp_decode_qk_rope_cache_rows")
                c(L.bp_decode_attention_rows(self.vq.data_ptr(), kc.data_ptr(), vc.data_ptr(), self.v_pos.data_ptr(),
                                             self.vattn.data_ptr(), cfg.heads, cfg.head_dim, cfg.max_len, self.scale,
                                             s, st), "bp_decode_attention_rows")
            self._mm(self.vattn[:s], w["o"], self.vo[:s])
            if self._pro_fits(2 * F, H, s):
                self._pro_mm(self.vo[:s], w["gate_up"], self.vact[:s], w["post_attn"], res[:s], spare[:s], silu=True)
                res, spare = spare, res
            else:
                norm_into(self.vo, w["post_attn"])
                self._gate_up_silu(res[:s], w["gate_up"], self.vact, self.vgu, s)
            dc = self._down_splitk(s)
            if dc is not None:  # split-K partials; their reduce feeds the norm in one launch
                dw = w["down"]
                rb, waves, split, xs = dc
                c(L.bp_skinny_mf_partials(S._KIND_CODE[self.kind], self.vact.data_ptr(), dw[0].data_ptr(), s, H, F,
                                          rb, waves, split, xs, self.vws.data_ptr(), self.vws.numel() * 4, st),
                  "bp_skinny_mf_partials")
                sc, sdt = (dw[1].data_ptr(), _lib.TORCH_DT[dw[1].dtype]) if self.kind == "int8" else (None, 0)
                c(L.bp_decode_splitk_norm_residual_rows(self.vws.data_ptr(), split, sc, sdt, w["post_ff"].data_ptr(),
                                                        res.data_ptr(), res.data_ptr(), H, cfg.eps, s, st),
                  "bp_decode_splitk_norm_residual_rows")
            else:
                self._mm(self.vact[:s], w["down"], self.vdn[:s])
                pending = w["post_ff"]
        if pending is not None and self._pro_fits(V, H, s, norms=2):  # both norms inside the head's launch
            self._pro_mm(self.vdn[:s], self.lm_head, self.vlogits[:s], pending, res[:s], spare[:s], gamma2=self.norm)
        else:
            if pending is not None:
                norm_into(self.vdn, pending)
            if self._pro_fits(V, H, s):
                self._pro_mm(res[:s], self.lm_head, self.vlogits[:s], self.norm, None, None)
            else:
                c(L.bp_decode_norm_residual_rows(res.data_ptr(), self.norm.data_ptr(), None, self.vxn.data_ptr(), H,
                                                 cfg.eps, s, st), "bp_decode_norm_residual_rows")
                self._mm(self.vxn[:s], self.lm_head, self.vlogits[:s])
        c(L.bp_decode_argmax_rows(self.vlogits.data_ptr(), cfg.vocab, s, self.v_tok.data_ptr(),
                                  self.v_argmax_scratch.data_ptr(), st), "bp_decode_argmax_rows")
        c(L.bp_draft_verify_next(self.v_ids.data_ptr(), self.v_tok.data_ptr(), self.v_out.data_ptr(),
                                 self.v_pos.data_ptr(), s, self.smax, st), "bp_draft_verify_next")

    def argmax_failed(self) -> bool:
        """Whether an argmax launch since the decoder was made gave up waiting for one of its partials (its token
        is then not to be trusted); reads the error words of the argmax scratch (synchronises)."""
        rows = [self.argmax_scratch.view(-1, ARGMAX_ROW_WORDS)]
        if getattr(self, "smax", 0):
            rows.append(self.v_argmax_scratch.view(-1, ARGMAX_ROW_WORDS))
        return any(bool(r[:, ARGMAX_ERROR_WORD].any().item()) for r in rows)

    def check_argmax(self) -> None:
        """Raises RuntimeError when argmax_failed()."""
        if self.argmax_failed():
            raise RuntimeError("an argmax launch gave up waiting for a partial result: its token is not valid")

    def weight_bytes(self) -> int:
        """Bytes of the linears' weights (and scales) a step streams."""
        lins = [self.lm_head] + [w[n] for w in self.layers for n in ("qkv", "o", "gate_up", "down")]
        return sum(t.numel() * t.element_size() for args in lins for t in args)


def _loop(dec: OlmoDecoder, group: int, issue: Callable[[int, int], None], prepare: Callable[[], None] | None,
          slots: torch.Tensor):
    """The token loop. After the prompt, the steps run in groups of up to `group` steps; issue(g, n) enqueues group
    g (n steps, each followed by a copy of its token into pinned slot 2 (g % 2) + j). Groups are enqueued one ahead
    of the host: the host reads group g's tokens while the GPU runs group g + 1 (whose first step reads the last
    token on the device), so the GPU does not wait for the host between groups. The tokens are those of one step
    at a time; steps enqueued past the end (an EOS inside a group, or the group after it) compute tokens nobody
    reads and leave cache rows past the end, which a later generate overwrites before reading them (it refills the
    cache from position 0)."""
    slots_np = slots.numpy()
    done = [torch.cuda.Event(), torch.cuda.Event()]

    @torch.no_grad()
    def generate(inputs: torch.Tensor, generation_config=None, **kwargs) -> torch.Tensor:
        if inputs.dim() != 2 or inputs.shape[0] != 1 or kwargs.get("do_sample"):
            raise OptimizeError("minimal loop supports batch size 1 and greedy decoding only")
        max_new = int(kwargs["max_new_tokens"])
        eos = kwargs.get("eos_token_id")
        eos_ids = set([eos] if isinstance(eos, int) else (eos or []))
        L = inputs.shape[1]
        if L < 1 or max_new < 1:
            raise OptimizeError("need a prompt and at least one new token")
        if L + max_new > dec.cfg.max_len:
            raise OptimizeError(f"{L}+{max_new} tokens exceed the static cache ({dec.cfg.max_len})")
        ids = inputs[0].tolist()
        if min(ids) < 0 or max(ids) >= dec.cfg.vocab:
            raise OptimizeError("token id outside the vocabulary")
        dev = dec.device
        dec.pos.zero_()
        for t in ids:  # prefill one position at a time; the last step leaves the first new token in tok
            dec.tok.fill_(t)
            dec.step()
        slots[0].copy_(dec.tok[0], non_blocking=True)
        done[0].record()
        done[0].synchronize()
        new = [int(slots_np[0])]
        need = max_new - 1  # tokens still to come
        if new[0] not in eos_ids and need > 0:
            if prepare is not None:
                prepare()
            sizes = [min(group, need - s) for s in range(0, need, group)]

            def launch(g: int) -> None:
                issue(g, sizes[g])
                done[g % 2].record()

            launch(0)
            for g, n in enumerate(sizes):
                if g + 1 < len(sizes):
                    launch(g + 1)  # one group ahead of the host
                done[g % 2].synchronize()
                stop = False
                for j in range(n):
                    new.append(int(slots_np[2 * (g % 2) + j]))
                    if new[-1] in eos_ids:
                        stop = True
                        break
                if stop:
                    break
        dec.check_argmax()
        return torch.cat([inputs[0].to(dev), torch.tensor(new, dtype=torch.long, device=dev)]).unsqueeze(0)

    return generate


def make_generate(dec: OlmoDecoder):
    """The minimal loop (olmo.py:51-119): the decode step run eagerly, its token copied to pinned memory."""
    slots = torch.zeros(4, dtype=torch.long).pin_memory()

    def issue(g: int, n: int) -> None:
        for j in range(n):
            dec.step()
            slots[2 * (g % 2) + j].copy_(dec.tok[0], non_blocking=True)

    return _loop(dec, 1, issue, None, slots)


GRAPH_STEPS = 2  # decode steps per graph replay (one graph launch per two tokens)


def make_generate_graph(dec: OlmoDecoder):
    """The graph loop (olmo.py:122-219): the first decode captures the step (after three warm-up steps on a side
    stream, which run at positions L .. L + 2 and leave cache rows that the real steps overwrite before they are
    read) into graphs of GRAPH_STEPS steps and of one step, each step followed by the copy of its token into its
    pinned slot, one graph per slot pair; the tokens then come GRAPH_STEPS per replay, with one synchronize per
    replay and the next replay already enqueued."""
    state: dict = {}
    slots = torch.zeros(4, dtype=torch.long).pin_memory()

    def prepare() -> None:
        if "graphs" in state:
            return
        tok, pos = dec.tok.clone(), dec.pos.clone()
        s = torch.cuda.Stream(dec.device)
        s.wait_stream(torch.cuda.current_stream(dec.device))
        with torch.cuda.stream(s):
            for _ in range(3):  # initialise every kernel and allocation before the capture
                dec.step()
        torch.cuda.current_stream(dec.device).wait_stream(s)
        torch.cuda.synchronize(dec.device)
        graphs = {}
        for pair in (0, 1):
            for n in sorted({1, GRAPH_STEPS}):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for j in range(n):
                        dec.step()
                        slots[2 * pair + j].copy_(dec.tok[0], non_blocking=True)
                graphs[(pair, n)] = g
        state["graphs"] = graphs
        dec.tok.copy_(tok)
        dec.pos.copy_(pos)

    def issue(g: int, n: int) -> None:
        state["graphs"][(g % 2, n)].replay()

    return _loop(dec, GRAPH_STEPS, issue, prepare, slots)
