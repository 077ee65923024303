"""Which linear layers a quantization target selects (pure: module names in, bool out).

The selection is by module name, so it has to accept exactly the names the reference accepts
(byteprof/quant/select.py:25-60): OLMo 2 / Bolmo global layers `model.layers.<i>.self_attn.{q,k,v,o}_proj` and
`model.layers.<i>.mlp.{gate,up,down}_proj`; Bolmo local layers under `model.local_{encoder,decoder}.layers.<i>`
(xlstm q/k/v/ogate_preact/out_proj and the MLP) plus the encoder's out_projection and the decoder's
in_projection; `lm_head` only for the OLMo target "blocks+head". Embeddings, norms, the boundary predictor and
the mLSTM gate projections are never selected.
"""

from __future__ import annotations

import re

BOLMO_TARGETS = ("none", "local", "global", "all")
OLMO_TARGETS = ("blocks", "blocks+head")
VALID_TARGETS = BOLMO_TARGETS + OLMO_TARGETS
VALID_SCHEMES = ("int8_wo", "int4_wo")

_LAYER = r"\.layers\.\d+\."
_GLOBAL_RE = re.compile(r"^model" + _LAYER + r"(?:self_attn\.(?:q|k|v|o)_proj|mlp\.(?:gate|up|down)_proj)$")
_LOCAL_RE = re.compile(
    r"^model\.local_(?:encoder|decoder)" + _LAYER
    + r"(?:xlstm\.(?:q|k|v|ogate_preact|out_proj)|mlp\.(?:gate|up|down)_proj)$"
    + r"|^model\.local_encoder\.out_projection$|^model\.local_decoder\.in_projection$")


def group_of(module_name: str) -> str | None:
    """'local', 'global', or None for a linear that is never quantized (Bolmo naming)."""
    if _LOCAL_RE.match(module_name):
        return "local"
    if _GLOBAL_RE.match(module_name):
        return "global"
    return None


def should_quantize(module_name: str, target: str) -> bool:
    """Bolmo targets: none | local | global | all."""
    if target not in BOLMO_TARGETS:
        raise ValueError(f"Bolmo target must be one of {list(BOLMO_TARGETS)}, got {target!r}")
    g = group_of(module_name)
    return g is not None and target in ("all", g)


def olmo_group_of(module_name: str) -> str | None:
    """'blocks' for the linears of OLMo 2's transformer layers, 'head' for lm_head, else None."""
    if _GLOBAL_RE.match(module_name):
        return "blocks"
    return "head" if module_name == "lm_head" else None


def olmo_should_quantize(module_name: str, target: str) -> bool:
    """OLMo 2 targets: none | blocks | blocks+head."""
    if target not in ("none",) + OLMO_TARGETS:
        raise ValueError(f"OLMo target must be one of {['none', *OLMO_TARGETS]}, got {target!r}")
    g = olmo_group_of(module_name)
    if g == "blocks":
        return target in OLMO_TARGETS
    return g == "head" and target == "blocks+head"


def selects(target: str, group: str | None) -> bool:
    """Does `target` quantize a linear of this group (local, global, blocks, head)?"""
    if group is None or target == "none":
        return False
    allowed = {"local": ("local",), "global": ("global",), "all": ("local", "global"),
               "blocks": ("blocks",), "blocks+head": ("blocks", "head")}
    return group in allowed[target]
