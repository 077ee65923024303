"""GPU parity of the grouped skinny launch (optim/skinny_group.py, csrc/skinny_group.hip).

Each item's output is checked two ways: bitwise against skinny_mm at one activation row with the same waves and
split 1 (the same per-row arithmetic in the same order; the wave sum's addition tree does not depend on how many
rows a workgroup holds, so any rows value matches), and against the oracle (the componentwise and normwise gates
of the skinny tests). Output elements outside the items' rows keep their sentinels.
"""

from __future__ import annotations

import pytest
import torch

from byteprof_amd import decode_set as D
from byteprof_amd.optim.skinny import skinny_mm
from byteprof_amd.optim.skinny_group import DEFAULT_CFG, GroupItem, SkinnyGroup
from tests.helpers import check_against_oracle, make_weights, normwise, oracle_weights, randn_x, torch_reference

pytestmark = pytest.mark.gpu
DEV = "cuda"
SENTINEL = 1234.0  # exact in bf16
GAP = 8  # sentinel elements before and after every item's outputs

BF16_SHAPES = [(2048, 2048), (0, 1024), (3, 512), (1, 1536), (777, 1536), (8192, 512), (513, 8192), (2, 2048)]
INT8_SHAPES = [(2048, 2048), (0, 1024), (3, 1024), (1, 3072), (777, 2048), (8192, 1024), (513, 8192), (2, 2048)]


def _items(kind, shapes, seed, scale_dtype=None):
    """Seeded items whose outputs are views of one sentinel-filled buffer, GAP elements apart (odd offsets too)."""
    total = sum(n + 2 * GAP + 1 for n, _ in shapes)
    buf = torch.full((total,), SENTINEL, dtype=torch.bfloat16, device=DEV)
    items, args, off = [], [], 0
    for i, (n, k) in enumerate(shapes):
        _, a = make_weights(kind, n, k, seed=seed + i, scale_dtype=scale_dtype)
        x = randn_x(1, k, seed=seed + 100 + i)[0]
        y = buf[off + GAP + (i % 2):off + GAP + (i % 2) + n]
        off += n + 2 * GAP + 1
        items.append(GroupItem(x, a[0], y, a[1] if kind == "int8" else None))
        args.append(a)
    return items, args, buf


def _outside_untouched(items, buf):
    mask = torch.ones_like(buf, dtype=torch.bool)
    base = buf.data_ptr()
    for it in items:
        lo = (it.y.data_ptr() - base) // 2
        mask[lo:lo + it.y.numel()] = False
    assert bool((buf[mask] == SENTINEL).all())


def _check(kind, items, args, cfg):
    rows, waves = cfg
    for it, a in zip(items, args):
        n = it.w.shape[0]
        if n == 0:
            continue
        ref = skinny_mm(it.x[None], *a, cfg=(max(rows, 2), waves, 1))
        assert torch.equal(it.y.view(torch.int16), ref[0].view(torch.int16)), (tuple(it.w.shape), cfg)
        check_against_oracle(it.y[None], it.x[None], oracle_weights(kind, a))


@pytest.mark.parametrize("cfg", [(2, 4), (1, 4), (4, 2), (8, 1), (2, 8), (4, 4)])
def test_bf16_group_matches_skinny_mm_and_the_oracle(cfg):
    items, args, buf = _items("bf16", BF16_SHAPES, seed=10)
    SkinnyGroup(items, cfg=cfg).run()
    torch.cuda.synchronize()
    _check("bf16", items, args, cfg)
    _outside_untouched(items, buf)


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cfg", [DEFAULT_CFG["int8"], (4, 2), (2, 4), (1, 1)])
def test_int8_group_matches_skinny_mm_and_the_oracle(cfg, scale_dtype):
    items, args, buf = _items("int8", INT8_SHAPES, seed=20, scale_dtype=scale_dtype)
    SkinnyGroup(items, cfg=cfg).run()
    torch.cuda.synchronize()
    _check("int8", items, args, cfg)
    _outside_untouched(items, buf)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_decode_step_set_as_one_group(kind):
    """The 113 linears of the OLMo-2-1B decode step (2.56 GB bf16 / 1.28 GB int8), each on its own unit-RMS input:
    every output bitwise equal to its own skinny_mm call; the LM head also within the normwise gate of the fp32
    formulation."""
    ops = D.build(kind, 1, DEV, seed=3)
    group = D.group_of(ops)
    assert group.blocks == sum(-(-o.n // group.rows) for o in ops)
    for o in ops:
        o.y.fill_(SENTINEL)
    group.run()
    torch.cuda.synchronize()
    for o in ops:
        ref = skinny_mm(o.x, *o.args, cfg=(max(group.rows, 2), group.waves, 1))
        assert torch.equal(o.y.view(torch.int16), ref.view(torch.int16)), o.name
    head = ops[-1]
    w32 = head.args[0].float() if kind == "bf16" else head.args[0].float() * head.args[1].float()[:, None]
    assert normwise(head.y, torch_reference(head.x, w32)) < 1e-2


def test_group_replays_in_a_graph_match_eager_runs():
    items, args, buf = _items("bf16", BF16_SHAPES, seed=30)
    group = SkinnyGroup(items)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        group.run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        group.run()
    for rep in range(3):
        for i, it in enumerate(items):
            it.x.copy_(randn_x(1, it.x.numel(), seed=1000 * rep + i)[0])
        g.replay()
        torch.cuda.synchronize()
        got = [it.y.clone() for it in items]
        for it in items:
            it.y.fill_(SENTINEL)
        group.run()
        torch.cuda.synchronize()
        for a, it in zip(got, items):
            assert torch.equal(a.view(torch.int16), it.y.view(torch.int16)), rep
    _check("bf16", items, args, group_cfg := (group.rows, group.waves))
    assert group_cfg == DEFAULT_CFG["bf16"]


def test_group_rejects_bad_arguments():
    _, (w,) = make_weights("bf16", 64, 1024, seed=1)
    _, (q, s) = make_weights("int8", 64, 1024, seed=1, scale_dtype=torch.float16)
    x = randn_x(1, 1024, seed=2)[0]
    y = torch.empty(64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="at least one"):
        SkinnyGroup([])
    with pytest.raises(ValueError, match="multiple of 512"):
        SkinnyGroup([(x[:1000], w[:, :1000].contiguous(), y)])
    with pytest.raises(ValueError, match="16-byte aligned"):
        xb = torch.empty(1032, dtype=torch.bfloat16, device=DEV)
        SkinnyGroup([(xb[1:1025], w, y)])
    with pytest.raises(ValueError, match="contiguous bf16"):
        SkinnyGroup([(x.float(), w, y)])
    with pytest.raises(ValueError, match=r"y must be"):
        SkinnyGroup([(x, w, y[:63])])
    with pytest.raises(ValueError, match="same|must be contiguous"):
        SkinnyGroup([(x, w, y), (x, q, y, s)])
    with pytest.raises(ValueError, match="scale"):
        SkinnyGroup([(x, q, y)])
    with pytest.raises(ValueError, match="take no scale"):
        SkinnyGroup([(x, w, y, s)])
    with pytest.raises(ValueError, match="no compiled"):
        SkinnyGroup([(x, w, y)], cfg=(3, 4))
    with pytest.raises(ValueError, match="GPU"):
        SkinnyGroup([(x.cpu(), w.cpu(), y.cpu())])
