"""Drafting (speculative decoding) for the OLMo-2 decode loop: batch 1, greedy, static KV cache, one captured HIP
graph per draft length K.

Drop-in for byteprof/optim/olmo_draft.py (make_generate_draft): each round verifies K + 1 tokens [t0, d_1 .. d_K]
at cache positions p .. p + K in one graph replay (OlmoDecoder.verify: the rows' logits, their argmax, the accepted
length L on the device, the next round's t0 <- p_{L+1} and position p + L + 1), then one pinned read and one
synchronize; the host emits the L + 1 tokens and asks the drafter for the next drafts. Rollback of the KV cache is
that position: entries written beyond it are overwritten by the next round before any row reads them.

Drafters follow the reference's protocol (byteprof/drafting/drafters.py): reset(ctx, truth), propose(k) -> list of
up to k ids, push(emitted). Built in: 'none' (no drafts: every round is one decode step) and 'oracle' (the
recorded continuation: every draft is accepted; the upper bound of a drafter). The reference's n-gram and
prompt-lookup drafters plug into the same protocol (spec 'drafter').
"""

from __future__ import annotations

from typing import Any, Callable, Sequence

import torch

from .olmo import OlmoDecoder, OptimizeError


class NullDrafter:
    """No drafts (byteprof/drafting/drafters.py:14-24)."""

    name = "none"

    def reset(self, ctx: Sequence[int], truth: Sequence[int] | None = None) -> None:
        pass

    def propose(self, k: int) -> list[int]:
        return []

    def push(self, tokens: Sequence[int]) -> None:
        pass


class OracleDrafter:
    """The true next tokens (byteprof/drafting/drafters.py:27-45): truth[0] is the first generated token."""

    name = "oracle"

    def __init__(self) -> None:
        self.truth: Sequence[int] = []
        self.i = 0

    def reset(self, ctx: Sequence[int], truth: Sequence[int] | None = None) -> None:
        if truth is None:
            raise ValueError("the oracle drafter needs the ground-truth tokens")
        self.truth, self.i = truth, 0

    def propose(self, k: int) -> list[int]:
        return list(self.truth[self.i + 1:self.i + 1 + k])

    def push(self, tokens: Sequence[int]) -> None:
        self.i += len(tokens)


def accepted_length(ids: Sequence[int], toks: Sequence[int], k: int) -> int:
    """ids = [t0, d_1 .. d_K], toks = the K + 1 row predictions: the number of leading drafts equal to the
    prediction before them (byteprof/optim/draft_core.py:27-32)."""
    n = 0
    while n < k and ids[n + 1] == toks[n]:
        n += 1
    return n


def choose_k(draft_len: int, k_values: Sequence[int], k_cap: int) -> int:
    """Largest available K not above the draft length and the cap (byteprof/optim/draft_core.py:182-188)."""
    best = 0
    for kv in k_values:
        if kv <= draft_len and kv <= k_cap and kv > best:
            best = kv
    return best


class Stats:
    """Round statistics (byteprof/optim/draft_core.py:161-172, the fields this loop fills)."""

    def __init__(self) -> None:
        self.rounds = 0
        self.emitted = 0
        self.by_k: dict[int, int] = {}
        self.l_hist: dict[int, int] = {}

    def dump(self) -> dict:
        return {"rounds": self.rounds, "emitted": self.emitted, "by_k": dict(self.by_k), "l_hist": dict(self.l_hist),
                "tokens_per_round": self.emitted / max(self.rounds, 1)}


def build_drafter(spec: dict[str, Any]) -> Any:
    kind = spec.get("kind", "none")
    if "drafter" in spec:
        return spec["drafter"]
    if kind == "none":
        return NullDrafter()
    if kind == "oracle":
        return OracleDrafter()
    raise OptimizeError(f"unknown draft kind {kind!r} (built in: 'none', 'oracle'; or pass spec['drafter'])")


def make_generate_draft(dec: OlmoDecoder, spec: dict[str, Any] | None = None,
                        stats: Stats | None = None) -> tuple[Callable, dict]:
    """generate(inputs, max_new_tokens=..., eos_token_id=None) with drafting rounds; returns (generate, state).

    spec: 'kind' ('none' | 'oracle'), 'ks' (draft lengths with a captured graph, default (0, 1, 2, 4, 6, 8)), 'k_max'
    (default 8), 'truth' ({prompt ids tuple: generated tokens}, for 'oracle'), 'drafter' (any object with the
    protocol). The prompt is fed one position at a time through OlmoDecoder.step (as make_generate does), which
    also gives the first new token; the rounds then run from the end of the prompt."""
    spec = dict(spec or {})
    k_max = int(spec.get("k_max", 8))
    ks = (0,) + tuple(sorted(k for k in spec.get("ks", (0, 1, 2, 4, 6, 8)) if 0 < k <= k_max))
    smax = max(ks) + 1
    drafter = build_drafter(spec)
    truths = spec.get("truth")
    dec.verify_buffers(smax)
    dev = dec.device
    pinned_d = torch.zeros(smax, dtype=torch.long).pin_memory()
    pinned_o = torch.zeros(dec.smax + 1, dtype=torch.long).pin_memory()  # row tokens, accepted length at dec.smax
    pinned_one = torch.zeros(1, dtype=torch.long).pin_memory()
    d_np, o_np, one_np = pinned_d.numpy(), pinned_o.numpy(), pinned_one.numpy()
    done = torch.cuda.Event()
    st: dict[str, Any] = {"graphs": {}, "ks": ks, "smax": smax}

    def build() -> None:
        """Warm-up and capture of one graph per K. The warm-up rounds run from the current position (they write
        cache rows at and after it, which the real rounds overwrite before reading); the round inputs are restored."""
        ids, pos = dec.v_ids.clone(), dec.v_pos.clone()
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            for _ in range(2):
                for k in ks:
                    dec.verify(k + 1)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize(dev)
        for k in ks:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                dec.verify(k + 1)
            st["graphs"][k] = g
        torch.cuda.synchronize(dev)
        dec.v_ids.copy_(ids)
        dec.v_pos.copy_(pos)

    @torch.no_grad()
    def generate(inputs: torch.Tensor, generation_config: Any = None, **kwargs: Any) -> torch.Tensor:
        if inputs.dim() != 2 or inputs.shape[0] != 1 or kwargs.get("do_sample"):
            raise OptimizeError("the drafting loop supports batch size 1 and greedy decoding only")
        max_new = int(kwargs["max_new_tokens"])
        eos = kwargs.get("eos_token_id")
        eos_ids = set([eos] if isinstance(eos, int) else (eos or []))
        n_prompt = inputs.shape[1]
        if n_prompt < 1 or max_new < 1:
            raise OptimizeError("need a prompt and at least one new token")
        if n_prompt + max_new + smax > dec.cfg.max_len:
            raise OptimizeError(f"{n_prompt}+{max_new} tokens exceed the static cache ({dec.cfg.max_len})")
        ids = inputs[0].tolist()
        if min(ids) < 0 or max(ids) >= dec.cfg.vocab:
            raise OptimizeError("token id outside the vocabulary")
        dec.pos.zero_()
        for t in ids:  # prefill one position at a time; the last step leaves the first new token in tok
            dec.tok.fill_(t)
            dec.step()
        pinned_one.copy_(dec.tok, non_blocking=True)
        done.record()
        done.synchronize()
        new = [int(one_np[0])]
        if new[0] not in eos_ids and len(new) < max_new:
            dec.v_ids[:1].copy_(dec.tok)
            dec.v_pos.fill_(n_prompt)
            if not st["graphs"]:
                build()
            truth = None
            if truths is not None:
                truth = truths.get(tuple(ids))
                if truth is None:
                    raise OptimizeError("oracle drafter: no recorded continuation for this prompt")
            drafter.reset(ids + [new[0]], truth)
            last = new[0]
            while True:
                draft = drafter.propose(k_max) if k_max > 0 and len(ks) > 1 else []
                k = choose_k(len(draft), ks, k_max)
                if k:
                    d_np[:k] = draft[:k]
                    dec.v_ids[1:1 + k].copy_(pinned_d[:k], non_blocking=True)
                st["graphs"][k].replay()
                pinned_o.copy_(dec.v_out, non_blocking=True)
                done.record()
                done.synchronize()  # the single sync of this round
                toks = o_np[:k + 1].tolist()
                length = int(o_np[dec.smax])
                if length != accepted_length([last] + list(draft[:k]), toks, k):
                    raise RuntimeError("host and device disagree on the accepted length")
                emitted = toks[:length + 1]
                stop = False
                n_before = len(new)
                for r in emitted:
                    new.append(r)
                    if r in eos_ids or len(new) >= max_new:
                        stop = True
                        break
                if stats is not None:
                    stats.rounds += 1
                    stats.emitted += len(new) - n_before
                    stats.by_k[k] = stats.by_k.get(k, 0) + 1
                    stats.l_hist[length] = stats.l_hist.get(length, 0) + 1
                if stop:
                    break
                drafter.push(emitted)
                last = emitted[-1]
        dec.check_argmax()
        return torch.cat([inputs[0].to(dev), torch.tensor(new, dtype=torch.long, device=dev)]).unsqueeze(0)

    generate.drafter = drafter  # type: ignore[attr-defined]
    return generate, st
