"""Host-side logic of the drop-in modules on the CPU: module selection, byte accounting, the quantizer's bytes,
argument validation, configuration resolution and the CPU (dequantized) paths of the nn.Module drop-ins.
Selection / accounting cases follow byteprof tests/test_quant_accounting.py; validation follows
tests/test_skinny.py:125-132."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn as nn

from byteprof_amd.optim import skinny as S
from byteprof_amd.quant import accounting as A
from byteprof_amd.quant import select as SEL
from byteprof_amd.quant.hip_int8 import quantize_rowwise_int8
from oracle import numerics as ON
from oracle import skinny as OS

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- selection (names in, bool out) -----------------------------------------------------------------------------


def test_select_local_exactly():
    enc = "model.local_encoder.layers.0."
    dec = "model.local_decoder.layers.3."
    yes = [enc + s for s in ("xlstm.q", "xlstm.k", "xlstm.v", "xlstm.ogate_preact", "xlstm.out_proj",
                              "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")]
    yes += [dec + s for s in ("xlstm.q", "mlp.down_proj")]
    yes += ["model.local_encoder.out_projection", "model.local_decoder.in_projection"]
    no = ["lm_head", "model.local_encoder.byte_embedding", "model.local_encoder.subword_embedding",
          "model.local_encoder.boundary_predictor_module.q_proj_layer", enc + "xlstm.igate_preact",
          enc + "xlstm.fgate_preact", "model.local_decoder.layers", "model.local_encoder.layers.0.mlp",
          enc + "pre_xlstm_layernorm"]
    for n in yes:
        assert SEL.should_quantize(n, "local") and not SEL.should_quantize(n, "global") and SEL.should_quantize(n, "all")
        assert not SEL.should_quantize(n, "none")
    assert not SEL.should_quantize("model.layers.0.self_attn.q_proj", "local")
    for n in no:
        assert not any(SEL.should_quantize(n, t) for t in ("none", "local", "global", "all")), n


def test_select_global_and_olmo_targets():
    blocks = [f"model.layers.{i}.{s}" for i in (0, 15) for s in (
        "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")]
    for n in blocks:
        assert SEL.group_of(n) == "global" and SEL.should_quantize(n, "global")
        assert SEL.olmo_group_of(n) == "blocks"
        assert SEL.olmo_should_quantize(n, "blocks") and SEL.olmo_should_quantize(n, "blocks+head")
        assert not SEL.olmo_should_quantize(n, "none")
    assert SEL.olmo_group_of("lm_head") == "head"
    assert not SEL.olmo_should_quantize("lm_head", "blocks") and SEL.olmo_should_quantize("lm_head", "blocks+head")
    for n in ("model.layers.0.self_attn.q_norm", "model.layers.0", "model.embed_tokens", "model.layers.0.self_attn"):
        assert SEL.group_of(n) is None and SEL.olmo_group_of(n) is None
    with pytest.raises(ValueError):
        SEL.should_quantize("lm_head", "everything")
    with pytest.raises(ValueError):
        SEL.olmo_should_quantize("lm_head", "all")
    assert SEL.selects("blocks+head", "head") and not SEL.selects("blocks", "head") and not SEL.selects("none", "local")


# ---- byte accounting ----------------------------------------------------------------------------------------------


def test_linear_bytes_schemes():
    lin = A.Linear(8, 256, "local")
    assert A.linear_bytes(lin, None) == 8 * 256 * 2
    assert A.linear_bytes(lin, "int8_wo") == 8 * 256 + 8 * 2
    assert A.linear_bytes(lin, "int4_wo", 128) == 8 * 256 * 0.5 + 8 * 2 * 4
    with pytest.raises(ValueError):
        A.linear_bytes(A.Linear(8, 100), "int4_wo", 128)


def test_decode_set_byte_totals():
    """The algorithmic bytes of the OLMo-2-1B-shaped decode-step set at M = 1 (weights + activations + outputs)."""
    lins = [A.Linear(2048, 2048)] * 4 + [A.Linear(8192, 2048)] * 2 + [A.Linear(2048, 8192)]
    blocks = 16 * sum(A.call_bytes(l, None, 1) for l in lins)
    head = A.call_bytes(A.Linear(100352, 2048), None, 1)
    assert blocks + head == 2_560_237_568
    assert A.call_bytes(A.Linear(8192, 2048), None, 1) == 33_574_912
    int8 = 16 * sum(A.call_bytes(l, "int8_wo", 1) for l in lins) + A.call_bytes(A.Linear(100352, 2048), "int8_wo", 1)
    assert int8 == 1_282_027_520


# ---- quantizer bytes ----------------------------------------------------------------------------------------------


def test_quantizer_matches_the_exact_fixture():
    cases = json.loads((GOLDEN / "quantizer_kat.json").read_text())["cases"]
    for c in cases:
        w = torch.tensor([c["w"]], dtype=torch.bfloat16)
        sdt = torch.bfloat16 if c["scale_dtype"] == "bf16" else torch.float16
        q, s = quantize_rowwise_int8(w, sdt)
        assert q[0].tolist() == c["q"] and float(s[0]) == c["scale"] and s.dtype == sdt, c


def test_quantizer_matches_the_oracle_bit_for_bit():
    torch.manual_seed(0)
    w = (torch.randn(64, 512) * 0.02).to(torch.bfloat16)
    q, s = quantize_rowwise_int8(w)
    oq, os_ = OS.quantize_rowwise_int8(w.float().numpy(), "bf16")
    assert np.array_equal(q.numpy(), oq) and np.array_equal(s.float().numpy(), os_)
    assert q.dtype == torch.int8 and s.dtype == torch.bfloat16 and q.is_contiguous()


# ---- validation and configuration ---------------------------------------------------------------------------------


def test_skinny_mm_validation_errors():
    w = torch.zeros(8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 64, dtype=torch.bfloat16), w)  # K mismatch
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, dtype=torch.bfloat16)[:, ::2], w)  # not contiguous
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, dtype=torch.bfloat16), torch.zeros(8, 128, dtype=torch.int8))  # no scale
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, dtype=torch.bfloat16), torch.zeros(8, 128, dtype=torch.float64))
    with pytest.raises(ValueError):
        S.skinny_mm(torch.zeros(2, 128, dtype=torch.bfloat16), w)  # on the CPU: no CPU path
    with pytest.raises(ValueError):  # int4 on the CPU: no CPU path
        S.skinny_mm(torch.zeros(2, 256, dtype=torch.bfloat16), torch.zeros(1, 2, 32, 64, dtype=torch.uint8),
                    torch.zeros(2, 32, dtype=torch.bfloat16), torch.zeros(2, 32, dtype=torch.float16))
    with pytest.raises(ValueError):  # int4 with K not a multiple of the group
        S.skinny_mm(torch.zeros(2, 200, dtype=torch.bfloat16), torch.zeros(1, 2, 32, 64, dtype=torch.uint8),
                    torch.zeros(2, 32, dtype=torch.bfloat16), torch.zeros(2, 32, dtype=torch.float16))
    with pytest.raises(ValueError):  # int4 without zero
        S.skinny_mm(torch.zeros(2, 256, dtype=torch.bfloat16), torch.zeros(1, 2, 32, 64, dtype=torch.uint8),
                    torch.zeros(2, 32, dtype=torch.bfloat16))


def test_configuration_keeps_one_k_order_per_shape():
    """waves and split (the K order) must not depend on the row count: the tuned table and the heuristic give one
    (waves, split) per shape for every launch of 1..64 rows (the weight blocks and staging may differ)."""
    for kind in ("bf16", "int8"):
        for n, k in ((2048, 2048), (8192, 2048), (2048, 8192), (100352, 2048), (6144, 2048), (16384, 2048),
                     (37, 256), (129, 640), (8, 5000)):
            orders = {S._resolve(kind, n, k, m, None)[1:3] for m in (1, 2, 4, 5, 8, 9, 16, 17, 32, 33, 64)}
            assert len(orders) == 1, (kind, n, k, orders)


def test_reference_cfg_tuples_are_mapped():
    """(BN, BK, warps, stages[, split]) and (rows, waves, split) map onto (weight blocks, waves, split, staging)."""
    assert S._resolve("bf16", 192, 1024, 1, (32, 128, 4, 3, 4)) == (4, 4, 4, 0)
    assert S._resolve("bf16", 192, 1024, 16, (64, 64, 2, 2, 1)) == (4, 2, 1, 0)  # rows clamped to the menu
    assert S._resolve("bf16", 192, 1024, 33, (64, 64, 2, 2, 1)) == (2, 2, 1, 0)  # 4 blocks only up to 16 rows
    assert S._resolve("int8", 192, 1024, 1, (16, 256, 4, 3, 3)) == (2, 4, 3, 0)
    assert S._resolve("bf16", 192, 1024, 1, (4, 8, 2)) == (1, 8, 2, 0)
    with pytest.raises(ValueError):
        S._resolve("bf16", 192, 1024, 1, (1, 2))


# ---- CPU paths of the drop-in modules (the reference's dequantized F.linear path) -------------------------------


def test_skinny_linear_cpu_inputs_use_the_dequantized_weights():
    from byteprof_amd.optim.skinny_linear import SkinnyLinear

    torch.manual_seed(1)
    lin = nn.Linear(256, 64, bias=True, dtype=torch.float32)
    m = SkinnyLinear(lin, "int8_wo")
    assert m.weight.numel() == 0 and m.weight.dtype == torch.float32
    x = torch.randn(3, 256)
    y = m(x)
    assert torch.allclose(y, x @ m.dequantized(torch.float32).T + lin.bias, atol=1e-5, rtol=1e-5)
    assert m(x.new_empty(0, 256)).shape == (0, 64)
    with pytest.raises(ValueError):
        SkinnyLinear(lin, "int3_wo")
    m4 = SkinnyLinear(lin, "int4_wo")  # fp32 weights: scale in fp32, zero in fp16
    y4 = m4(x)
    assert torch.allclose(y4, x @ m4.dequantized(torch.float32).T + lin.bias, atol=1e-5, rtol=1e-5)


class _Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.self_attn = nn.ModuleDict({n: nn.Linear(d, d, bias=False) for n in ("q_proj", "k_proj", "v_proj", "o_proj")})
        self.mlp = nn.ModuleDict({"gate_proj": nn.Linear(d, 2 * d, bias=False), "up_proj": nn.Linear(d, 2 * d, bias=False),
                                  "down_proj": nn.Linear(2 * d, d, bias=False)})


class _Toy(nn.Module):
    def __init__(self, d=256):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([_Block(d) for _ in range(2)])
        self.lm_head = nn.Linear(d, 64, bias=False)


@pytest.mark.parametrize("scheme,kernel", [("bf16_wo", "skinny"), ("int8_wo", "skinny"), ("int8_wo", "default")])
def test_apply_quantization_swaps_the_selected_linears(scheme, kernel):
    from byteprof_amd.optim.skinny_linear import SkinnyLinear
    from byteprof_amd.quant.integrate import Int8Linear, apply_quantization

    torch.manual_seed(0)
    m = _Toy().to(torch.bfloat16)
    stats = apply_quantization(m, "blocks", scheme, 128, None, None, kernel)
    cls = SkinnyLinear if kernel == "skinny" else Int8Linear
    assert stats["n_linears"] == 14 and sum(isinstance(x, cls) for x in m.modules()) == 14
    assert isinstance(m.lm_head, nn.Linear)
    assert ("kernel" in stats) == (kernel != "default")
    m2 = _Toy().to(torch.bfloat16)
    assert apply_quantization(m2, "blocks+head", scheme, 128, None, None, kernel)["n_linears"] == 15


def test_default_kernel_rejects_the_skinny_only_scheme():
    from byteprof_amd.quant.integrate import apply_quantization

    with pytest.raises(ValueError):
        apply_quantization(_Toy(), "blocks", "bf16_wo")


def test_int8linear_cpu_path_matches_dequantized_reference():
    from byteprof_amd.quant.integrate import Int8Linear

    torch.manual_seed(2)
    lin = nn.Linear(128, 32, bias=True, dtype=torch.bfloat16)
    mod = Int8Linear(lin)
    x = torch.randn(2, 1, 128, dtype=torch.bfloat16)
    y = mod(x)
    ref = torch.nn.functional.linear(x.reshape(2, 128), mod.q.to(torch.bfloat16) * mod.scale[:, None], lin.bias)
    assert y.shape == (2, 1, 32) and torch.equal(y.reshape(2, 32), ref)


def test_multistep_fw_validation():
    from byteprof_amd.optim import draft_fused as F

    nh, dq, dv, t = 2, 48, 16, 3
    cur = (torch.zeros(1, nh, dq, dv), torch.zeros(1, nh, dq), torch.zeros(1, nh, 1))
    q = torch.zeros(t, nh, dq)
    v = torch.zeros(t, nh, dv)
    g = torch.zeros(t, nh, 1)
    with pytest.raises(NotImplementedError):  # DQ not a multiple of 64
        F.multistep_fw(cur, q, q, v, g, g, torch.zeros(t, nh, dv), torch.zeros(nh, dq), torch.zeros(nh), 1e-6)
    dq = 64
    cur = (torch.zeros(1, nh, dq, dv), torch.zeros(1, nh, dq), torch.zeros(1, nh, 1))
    q = torch.zeros(t, nh, dq)
    with pytest.raises(ValueError):  # GPU only
        F.multistep_fw(cur, q, q, v, g, g, torch.zeros(t, nh, dv), torch.zeros(nh, dq), torch.zeros(nh), 1e-6)
    with pytest.raises(ValueError):  # h too short
        F.multistep_fw(cur, q, q, v, g, g, torch.zeros(t - 1, nh, dv), torch.zeros(nh, dq), torch.zeros(nh), 1e-6)


def test_bf16_of_torch_matches_the_oracle_rounding():
    """torch's .to(bfloat16) (what every drop-in output is compared in) rounds like the oracle."""
    x = torch.randn(5000) * 10
    assert np.array_equal(x.to(torch.bfloat16).float().numpy(), ON.bf16_round(x.numpy()))


def test_linear_chain_host_validation():
    """LinearChain checks kinds, shapes, inputs and dependencies before touching the GPU (CPU tensors here)."""
    from byteprof_amd.optim.linear_chain import ChainStage, LinearChain

    w = torch.zeros(64, 1024, dtype=torch.bfloat16)
    x = torch.zeros(1024, dtype=torch.bfloat16)
    out = torch.empty(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        LinearChain([])
    with pytest.raises(ValueError):  # no kernel for 3 waves
        LinearChain([ChainStage([w], x, out)], waves=3)
    with pytest.raises(ValueError):  # reads a later stage
        LinearChain([ChainStage([w], (1, 0), out), ChainStage([w], x, torch.empty(64, dtype=torch.bfloat16))])
    with pytest.raises(ValueError):  # the slice runs past the producer's output
        LinearChain([ChainStage([w], x, out), ChainStage([w], (0, 0), torch.empty(64, dtype=torch.bfloat16))])
    with pytest.raises(ValueError):  # the input is not bf16
        LinearChain([ChainStage([w], x.float(), out)])
    with pytest.raises(ValueError):  # mixed weight kinds
        q, sc = quantize_rowwise_int8(w)
        LinearChain([ChainStage([w], x, out), ChainStage([(q, sc)], x, torch.empty(64, dtype=torch.bfloat16))])
    with pytest.raises(ValueError):  # out holds fewer rows than the weights
        LinearChain([ChainStage([w, w], x, out)])
    from byteprof_amd._lib import NativeError
    with pytest.raises(NativeError):  # K not a multiple of the 64-element segment: refused by the plan
        LinearChain([ChainStage([torch.zeros(8, 100, dtype=torch.bfloat16)], torch.zeros(100, dtype=torch.bfloat16),
                                torch.empty(8, dtype=torch.bfloat16))])


def test_decode_chain_structure():
    """The decode-step chain on CPU tensors (structure only): 65 stages, each dependent stage reading the output
    a decode step feeds it, and the same byte total as the per-launch set."""
    from byteprof_amd import decode_set as D

    weights = {name: (torch.zeros(n, k, dtype=torch.bfloat16),) for name, n, k in D.shapes()}
    stages = D.chain_stages(weights, dependent=True, device="cpu")
    assert len(stages) == 65
    assert isinstance(stages[0].src, torch.Tensor)
    for i, st in enumerate(stages[1:], start=1):
        assert isinstance(st.src, tuple) and st.renorm
    assert [len(st.weights) for st in stages[:4]] == [3, 1, 2, 1]
    assert stages[1].src == (0, 2 * 2048)      # o reads v: rows 4096..6143 of q|k|v
    assert stages[2].src == (1, 0)             # gate|up reads o
    assert stages[3].src == (2, 8192)          # down reads up: rows 8192..16383 of gate|up
    assert stages[3].weights[0].shape == (2048, 8192)
    assert stages[4].src == (3, 0)             # the next layer's q|k|v reads down
    assert stages[-1].out.numel() == 100352 and stages[-1].src == (63, 0)
    ind = D.chain_stages(weights, dependent=False, device="cpu")
    assert len(ind) == 65 and all(isinstance(st.src, torch.Tensor) and not st.renorm for st in ind)
    assert D.chain_bytes("bf16") == 2_560_237_568 and D.chain_bytes("int8") == 1_282_027_520


def test_int4_quantizer_and_packing_match_the_oracle():
    """The host-side int4 format (torch, CPU) equals the oracle's restatement byte for byte."""
    from oracle import skinny as OS

    g = torch.Generator().manual_seed(7)
    for n, k, rows in ((37, 256, 32), (16, 384, 16), (70, 128, 64)):
        w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
        packed, scale, zero = S.quantize_int4(w, rows)
        assert packed.dtype == torch.uint8 and scale.dtype == torch.bfloat16 and zero.dtype == torch.float16
        p_o, s_o, z_o = OS.quantize_int4(w.float().numpy(), rows)
        assert np.array_equal(packed.numpy(), p_o)
        assert np.array_equal(scale.float().numpy(), s_o) and np.array_equal(zero.float().numpy(), z_o)
        assert torch.equal(S.unpack_int4(packed, n), torch.from_numpy(OS.unpack_int4(p_o, n)))
        deq = S.dequantize("int4", packed, scale, zero).numpy()
        assert np.allclose(deq, OS.dequantize_int4(p_o, s_o, z_o), rtol=0, atol=1e-7)


def test_int4_skinny_linear_holds_the_packed_format():
    from byteprof_amd.optim.skinny_linear import SkinnyLinear

    lin = torch.nn.Linear(256, 40, bias=False, dtype=torch.bfloat16)
    m = SkinnyLinear(lin, "int4_wo", tile_rows=32)  # the reference's packing
    assert m.q.shape == (2, 2, 32, 64) and m.scale.shape == (2, 40) and m.zero.shape == (2, 40)
    tuned = S.int4_tile_rows(40, 256)
    assert SkinnyLinear(lin, "int4_wo").q.shape == (-(-40 // tuned), 2, tuned, 64)
    with pytest.raises(ValueError):
        SkinnyLinear(lin, "int4_wo", tile_rows=48)
    assert m.weight.numel() == 0 and m.weight.dtype == torch.bfloat16
    x = torch.randn(3, 256, dtype=torch.bfloat16)
    y = m(x)  # CPU input: dequantized F.linear, as the reference
    assert torch.equal(y, torch.nn.functional.linear(x, m.dequantized(torch.bfloat16)))


def test_drafting_host_logic_matches_the_reference_definitions():
    """accepted_length / choose_k / the drafters, against hand-worked cases of the reference's definitions
    (byteprof/optim/draft_core.py:27-37,182-188; byteprof/drafting/drafters.py:14-45)."""
    from byteprof_amd.optim import olmo_draft as OD

    # drafts ids[1..k] against the predictions toks[0..k-1]; the first mismatch ends the count
    assert OD.accepted_length([9, 1, 2, 3], [1, 2, 3, 4], 3) == 3
    assert OD.accepted_length([9, 1, 2, 3], [1, 5, 3, 4], 3) == 1
    assert OD.accepted_length([9, 1, 2, 3], [7, 2, 3, 4], 3) == 0
    assert OD.accepted_length([9, 1, 2, 3], [1, 2, 3, 4], 2) == 2  # only k drafts count
    assert OD.accepted_length([9], [4], 0) == 0
    # the same count as the reference's device form: cumprod of the matches, summed
    rng = np.random.default_rng(0)
    for _ in range(200):
        k = int(rng.integers(0, 9))
        ids = rng.integers(0, 3, k + 1).tolist()
        toks = rng.integers(0, 3, k + 1).tolist()
        m = torch.tensor([ids[j + 1] == toks[j] for j in range(k)], dtype=torch.int32)
        want = int(torch.cumprod(m, 0).sum()) if k else 0
        assert OD.accepted_length(ids, toks, k) == want
    # the largest available K not above the draft length and the cap
    ks = (0, 1, 2, 4, 6, 8)
    assert [OD.choose_k(n, ks, 8) for n in range(10)] == [0, 1, 2, 2, 4, 4, 6, 6, 8, 8]
    assert OD.choose_k(9, ks, 5) == 4
    # the oracle drafter proposes the continuation after what it has been told was emitted
    d = OD.OracleDrafter()
    d.reset([1, 2, 3], truth=[50, 51, 52, 53, 54])
    assert d.propose(2) == [51, 52]
    d.push([51, 52])  # a round that emitted two tokens after t0 = truth[0]
    assert d.propose(8) == [53, 54]
    with pytest.raises(ValueError):
        OD.OracleDrafter().reset([1], None)
    assert OD.NullDrafter().propose(4) == []


def test_decode_stages_cover_the_linears():
    """The 65 stages are the 113 linears grouped by shared input (q|k|v, o, gate|up, down per layer, the head), in
    decode order, with the same bytes."""
    from byteprof_amd import decode_set as D

    stages = D.stage_shapes()
    assert len(stages) == 65 and [key for key, _, _ in stages] == D.stage_keys()
    assert stages[:4] == [("l0.qkv", 6144, 2048), ("l0.o", 2048, 2048), ("l0.gateup", 16384, 2048),
                          ("l0.down", 2048, 8192)]
    assert stages[-1] == ("lm_head", 100352, 2048)
    assert sum(n * k for _, n, k in stages) == sum(n * k for _, n, k in D.shapes())
    # algorithmic bytes of the 65 launches: weights (+ scales) once, inputs once per stage, outputs once
    stage_bytes = sum(A.call_bytes(A.Linear(n, k), None, 1) for _, n, k in stages)
    fewer_inputs = 2 * (2 * 2048 + 2048) * 16  # q|k|v read one input instead of three, gate|up one instead of two
    assert stage_bytes == D.chain_bytes("bf16") - fewer_inputs


def test_mlstm_head_dims_are_whole_waves():
    """DQ the fused mLSTM kernels take: multiples of 64 up to 256 (one row per thread) and 384 / 512 (two); 320 and
    448 would give workgroups of partial waves and are refused before any launch."""
    from byteprof_amd.optim import draft_fused as F

    assert [d for d in range(64, 640, 64) if F.supported_dq(d)] == [64, 128, 192, 256, 384, 512]
    q = torch.zeros(1, 2, 320)
    with pytest.raises(NotImplementedError):
        F._geometry(q, torch.zeros(1, 2, 16), 4)


# ---- the tuner's plan menu and table (byteprof_amd/tune.py) ------------------------------------------------------


def test_tuner_plans_cover_the_compiled_menu_and_skip_duplicates():
    """The tuner times (rb, xstage flags) plans that the library compiles: staging only where the rows fit the LDS
    stage, the general-loop flag only where a straight-line kernel of the segment count exists (elsewhere both
    flags run the same kernel)."""
    from byteprof_amd import tune as T

    fixed = list(T._plans("bf16", 1, 2048, 4, 1))    # 32 segments / 4 waves = 8 per wave: straight-line kernel
    assert {xs for _, xs in fixed} == {0, S.XS_STAGE, S.XS_GENERAL, S.XS_STAGE | S.XS_GENERAL}
    assert {rb for rb, _ in fixed} == {1, 2, 4}
    general = list(T._plans("bf16", 1, 2048, 1, 1))  # 32 segments per wave: the general loop only
    assert {xs for _, xs in general} == {0, S.XS_STAGE}
    big = list(T._plans("bf16", 33, 2048, 4, 1))      # more than 16 rows: no staging, 4 blocks only up to 16 rows
    assert {xs for _, xs in big} == {0, S.XS_GENERAL} and {rb for rb, _ in big} == {1, 2}
    assert all(S._supported("bf16", m, rb, w, xs & S.XS_STAGE)
               for m, w in ((1, 4), (1, 1), (33, 4)) for rb, xs in T._plans("bf16", m, 2048, w, 1))


def test_tuned_table_entries_resolve_to_compiled_plans():
    """Every bf16 / int8 entry of the committed table names one K order (waves, split) and, per row bucket, a
    weight-block count and flags that the launch maps onto a compiled kernel; every int4 entry a valid plan."""
    table = json.loads(S._CFG_FILE.read_text())
    for key, e in table.items():
        if key.startswith("_"):
            continue
        kind, n, k = key.split("|")
        n, k = int(n), int(k)
        if kind == "int4":
            assert S.int4_tile_rows(n, k) == e["tile_rows"] in S.INT4_TILES
            waves, split = S.int4_cfg(n, k, e["tile_rows"])
            assert (waves, split) == (e["waves"], e["split"]) and waves in (1, 2, 4, 8) and 1 <= split <= k // 128
            for rows, plan in e["tiles"].items():
                assert S.int4_cfg(n, k, int(rows)) == (plan["waves"], plan["split"])
            continue
        assert e["waves"] in (1, 2, 4, 8) and e["split"] >= 1
        for bucket in ("1", "8", "16", "32", "64"):
            xs = int(e["xs"][bucket])
            assert int(e["rb"][bucket]) in (1, 2, 4) and xs in (0, 1, 2, 3, 5, 9)
            # row groups: staged 9..16-row plans only
            assert not xs & S.XS_ROWS or (bucket == "16" and xs & S.XS_STAGE)
        for m in (1, 5, 8, 9, 16, 17, 33, 64):
            rb, waves, split, xs = S._resolve(kind, n, k, m, None)
            assert (waves, split) == (e["waves"], e["split"])
            assert S._supported(kind, m, rb, waves, xs & (S.XS_STAGE | S.XS_ROWS))
            if m in (9, 16):  # the table's plan is the one launched (no silent fallback)
                assert (rb, xs) == (int(e["rb"]["16"]), int(e["xs"]["16"])), (kind, n, k, m)
        # rb_pro (norm-prologue launches): only where the order keeps whole rows, for buckets 1 and 8, compiled,
        # and the one picked for those launches (same K order)
        assert set(e.get("rb_pro", {})) <= {"1", "8"} and (not e.get("rb_pro") or e["split"] == 1)
        for bucket, m in (("1", 1), ("8", 4)):
            if bucket in e.get("rb_pro", {}):
                rb, waves, split, _ = S._resolve(kind, n, k, m, None, pro=True)
                assert rb == int(e["rb_pro"][bucket]) and (waves, split) == (e["waves"], e["split"])
                assert S._supported(kind, m, rb, waves, True)


def test_every_mutant_plants_its_text_once():
    """The mutation check (tests/mutation.py) plants each bug by replacing one exact piece of source text: every
    piece must still occur exactly once, or the mutant would silently stop being built."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("mutation", Path(__file__).with_name("mutation.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    pkg = Path(__file__).resolve().parent.parent / "byteprof_amd"
    for name, rel, old, new in mod.MUTANTS:
        if new is None:
            continue
        assert (pkg / rel).read_text().count(old) == 1, name
