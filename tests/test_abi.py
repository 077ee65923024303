"""The C ABI: libbyteprof_amd.so loads (sharing torch's HIP runtime), exports every function include/byteprof_amd.h
declares, and rejects bad arguments before touching the GPU. CPU only: no call here launches a kernel."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "byteprof_amd.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(bp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from byteprof_amd import _lib

    return _lib.lib()


def test_header_declares_the_expected_entry_points():
    names = declared_functions()
    for required in ("bp_skinny_bf16", "bp_skinny_int8", "bp_gemv_int8", "bp_splitk_reduce", "bp_mlstm_multistep",
                     "bp_skinny_workspace_bytes", "bp_skinny_config_supported", "bp_version", "bp_status_string",
                     "bp_linear_set_run", "bp_linear_set_validate", "bp_linear_set_scratch_bytes",
                     "bp_linear_set_workgroups"):
        assert required in names


def test_library_exports_every_declared_symbol(L):
    for name in declared_functions():
        assert hasattr(L, name), name


def test_python_binding_covers_every_declared_symbol():
    from byteprof_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_one_hip_runtime_is_mapped(L):
    from byteprof_amd import _lib

    assert len(_lib._mapped_hip_runtimes()) <= 1


def test_version_and_status_strings(L):
    assert L.bp_version() >= 100
    for code in (0, -1, -2, -3):
        assert L.bp_status_string(code)
    assert b"workspace" in L.bp_status_string(-3)


def test_workspace_bytes(L):
    assert L.bp_skinny_workspace_bytes(4, 100, 1) == 0
    assert L.bp_skinny_workspace_bytes(4, 100, 3) == 3 * 4 * 100 * 4
    assert L.bp_skinny_workspace_bytes(0, 100, 3) == 0


def test_config_menu(L):
    # rows = 2 exists at every waves <= 8 for every row bucket and kind (one K order serves all buckets)
    for kind in (0, 1):
        for mt in (1, 2, 4, 8, 16):
            for waves in (1, 2, 4, 8):
                assert L.bp_skinny_config_supported(kind, mt, 2, waves), (kind, mt, waves)
    assert not L.bp_skinny_config_supported(0, 1, 3, 4)  # rows must be a power of two in the menu
    assert not L.bp_skinny_config_supported(0, 3, 2, 4)  # row buckets are 1, 2, 4, 8, 16
    assert not L.bp_skinny_config_supported(2, 1, 2, 4)  # kinds are 0 (bf16) and 1 (int8)


def test_invalid_arguments_are_rejected_before_any_launch(L):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below returns before enqueueing anything
    assert L.bp_skinny_bf16(None, p, p, 1, 1, 1, 4, 4, 1, None, 0, None) == -1       # null x
    assert L.bp_skinny_bf16(p, p, p, -1, 1, 1, 4, 4, 1, None, 0, None) == -1          # negative M
    assert L.bp_skinny_bf16(p, p, p, 17, 1, 1, 4, 4, 1, None, 0, None) == -1          # more than 16 rows
    assert L.bp_skinny_bf16(p, p, p, 0, 5, 5, 4, 4, 1, None, 0, None) == 0            # M = 0: no-op
    assert L.bp_skinny_bf16(p, p, p, 3, 0, 5, 4, 4, 1, None, 0, None) == 0            # N = 0: no-op
    assert L.bp_skinny_bf16(p, p, p, 1, 8, 1024, 3, 4, 1, None, 0, None) == -2        # rows not in the menu
    assert L.bp_skinny_bf16(p, p, p, 1, 8, 4096, 4, 4, 2, None, 0, None) == -3        # split without workspace
    assert L.bp_skinny_int8(p, p, None, 0, p, 1, 8, 64, 4, 4, 1, None, 0, None) == -1  # int8 without scale
    assert L.bp_skinny_int8(p, p, p, 7, p, 1, 8, 64, 4, 4, 1, None, 0, None) == -1     # bad scale dtype
    assert L.bp_splitk_reduce(None, p, None, 0, 2, 2, 2, None) == -1
    # mLSTM: DQ not a multiple of 64, bad value block, DV not a multiple of it
    args = [p] * 11
    assert L.bp_mlstm_multistep(*args, 4, 2, 48, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == -2
    assert L.bp_mlstm_multistep(*args, 4, 2, 64, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 5, None) == -2
    assert L.bp_mlstm_multistep(*args, 4, 2, 64, 12, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == -2
    assert L.bp_mlstm_multistep(*args, 4, 0, 64, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == 0  # NH = 0: no-op


def _set_stages(n_stages=2, k=2048, n=4096, kind=0):
    from byteprof_amd.optim.linear_set import BpSetStage

    arr = (BpSetStage * n_stages)()
    for i, h in enumerate(arr):
        h.src, h.y, h.x_used = (0x1000 if i == 0 else 0x2000), 0x2000, None
        h.K, h.N, h.wait_stage, h.renorm, h.nseg = k, n, i - 1, 1, 1
        h.seg_end[0] = n
        h.w[0] = 0x3000
        h.scale[0] = 0x4000 if kind == 1 else None
    return arr


def test_linear_set_descriptor_layout_matches_the_header():
    from byteprof_amd.optim.linear_set import BpSetStage

    text = HEADER.read_text()
    body = text[text.index("typedef struct BpSetStage"):text.index("} BpSetStage;")]
    fields = re.findall(r"^\s+[a-z_0-9 ]+?\*?\s*([a-z_A-Z]+)(?:\[\d\])?;", body, flags=re.M)
    assert fields == [f[0] for f in BpSetStage._fields_]
    assert ctypes.sizeof(BpSetStage) == 128


def test_linear_set_validation_rejects_bad_descriptors(L):
    """bp_linear_set_validate reads only the host descriptors: no GPU needed (the pointers are never used)."""
    def rc(arr, kind=0, groups=256, n=None):
        return L.bp_linear_set_validate(ctypes.addressof(arr), len(arr) if n is None else n, kind, groups)

    assert rc(_set_stages()) == 0
    assert rc(_set_stages(kind=1), kind=1) == 0
    assert rc(_set_stages(), n=0) == -1                      # no stages
    assert rc(_set_stages(), kind=2) == -2                   # unknown weight kind
    assert rc(_set_stages(k=1000)) == -2                     # K not a multiple of the 512-element chunk
    assert rc(_set_stages(k=1536), kind=1) == -2             # int8: K a multiple of 1024
    assert rc(_set_stages(k=16384)) == -2                    # input longer than the LDS buffer
    assert rc(_set_stages(n=512 * 256)) == -2                # more rows per workgroup than LDS holds
    assert rc(_set_stages(kind=0), kind=1) == -1             # int8 without scales
    bad = _set_stages()
    bad[1].wait_stage = 1                                    # a stage cannot wait for itself
    assert rc(bad) == -1
    bad = _set_stages()
    bad[0].seg_end[0] = 100                                  # segments must cover N
    assert rc(bad) == -1
    bad = _set_stages()
    bad[0].src = 0x1008                                      # inputs must be 16-byte aligned
    assert rc(bad) == -1
    bad = _set_stages()
    bad[0].nseg = 5
    assert rc(bad) == -1
    assert rc(_set_stages(n_stages=100)) == -2               # more stages than the LDS tables hold
    bad = _set_stages()
    bad[1].src = 0x2000 + 2 * 4096 - 16                      # a dependent input must lie inside its source's y
    assert rc(bad) == -1
    bad = _set_stages()
    bad[0].y = 0x2008                                        # outputs must be 16-byte aligned
    assert rc(bad) == -1
    arr = _set_stages(n_stages=3, n=4093)
    # launch counter + error flag lines, 3 x (4093 rounded up to 8) tagged rows
    assert L.bp_linear_set_scratch_bytes(ctypes.addressof(arr), 3, 256) == 4 * (64 + 3 * 4096)
    assert L.bp_linear_set_scratch_bytes(None, 0, 256) == 0


def _group_items(shapes, kind=0):
    from byteprof_amd.optim.skinny_group import BpGroupItem

    arr = (BpGroupItem * len(shapes))()
    for i, (h, (n, k)) in enumerate(zip(arr, shapes)):
        h.x, h.w, h.y = 0x10000 * (i + 1), 0x100000 * (i + 1), 0x1000000 * (i + 1)
        h.scale = 0x2000000 if kind == 1 else None
        h.N, h.K, h.block0 = n, k, -7
    return arr


def test_group_descriptor_layout_matches_the_header():
    from byteprof_amd.optim.skinny_group import LUT_SPAN, BpGroupItem

    text = HEADER.read_text()
    body = text[text.index("typedef struct BpGroupItem"):text.index("} BpGroupItem;")]
    fields = re.findall(r"^\s+[a-z_0-9 ]+?\*?\s*([a-z_A-Z0-9]+);", body, flags=re.M)
    assert fields == [f[0] for f in BpGroupItem._fields_]
    assert ctypes.sizeof(BpGroupItem) == 48
    assert f"#define BP_GROUP_LUT_SPAN {LUT_SPAN}" in text


@pytest.mark.parametrize("rows", [1, 2, 4, 8])
def test_group_plan_matches_a_brute_force_assignment(L, rows):
    """block0 is the running sum of ceil(N / rows); lut[j] is the item holding workgroup 256 j, found here by
    assigning every workgroup to its item one by one (items of 0 rows take none, tiny items share a span)."""
    shapes = [(2048, 2048), (0, 512), (3, 512), (1, 1024), (8192, 2048), (0, 512), (700, 8192), (5, 512),
              (100352, 2048), (0, 1024)]
    arr = _group_items(shapes)
    owner = [i for i, (n, _) in enumerate(shapes) for _ in range(-(-n // rows))]
    lut = (ctypes.c_int32 * 4096)()
    blocks = L.bp_skinny_group_plan(ctypes.addressof(arr), len(arr), 0, rows, ctypes.addressof(lut), len(lut))
    assert blocks == len(owner)
    starts = [sum(-(-n // rows) for n, _ in shapes[:i]) for i in range(len(shapes))]
    assert [h.block0 for h in arr] == starts
    spans = -(-blocks // 256)
    assert list(lut[:spans]) == [owner[256 * j] for j in range(spans)]
    # the kernel's walk from lut[b / 256] reaches the owner of every workgroup
    for b in range(blocks):
        g = lut[b // 256]
        while g + 1 < len(arr) and arr[g + 1].block0 <= b:
            g += 1
        assert g == owner[b], b
    # counting only (no lut)
    assert L.bp_skinny_group_plan(ctypes.addressof(arr), len(arr), 0, rows, None, 0) == blocks


def test_group_plan_and_run_reject_bad_items_before_any_launch(L):
    def plan(arr, kind=0, rows=2, cap=64):
        lut = (ctypes.c_int32 * cap)()
        return L.bp_skinny_group_plan(ctypes.addressof(arr), len(arr), kind, rows, ctypes.addressof(lut), cap)

    assert plan(_group_items([(64, 512)])) == 32
    assert plan(_group_items([(64, 1024)], kind=1), kind=1) == 32
    assert plan(_group_items([(64, 1000)])) == -1               # K not a multiple of the 512-element chunk
    assert plan(_group_items([(64, 1536)], kind=1), kind=1) == -1  # int8: K a multiple of 1024
    assert plan(_group_items([(64, 0)])) == -1                  # K = 0
    assert plan(_group_items([(-1, 512)])) == -1                # negative N
    assert plan(_group_items([(64, 512)]), kind=1) == -1        # int8 without scales
    assert plan(_group_items([(64, 512)]), kind=2) == -2        # unknown weight kind
    assert plan(_group_items([(64, 512)]), rows=0) == -1
    assert plan(_group_items([(2 * 256 * 64 + 2, 512)]), cap=64) == -1  # lut too small (65 spans)
    bad = _group_items([(64, 512)])
    bad[0].x = 0x10008                                          # x must be 16-byte aligned
    assert plan(bad) == -1
    bad = _group_items([(64, 512)])
    bad[0].w = None
    assert plan(bad) == -1
    assert L.bp_skinny_group_plan(None, 0, 0, 2, None, 0) == -1
    assert L.bp_skinny_group_config_supported(0, 2, 4) == 1
    assert L.bp_skinny_group_config_supported(1, 8, 8) == 1
    assert L.bp_skinny_group_config_supported(0, 3, 4) == 0
    assert L.bp_skinny_group_config_supported(0, 2, 16) == 0
    assert L.bp_skinny_group_config_supported(2, 2, 4) == 0

    arr = _group_items([(64, 512), (10, 512)])
    blocks = plan(arr)
    assert blocks == 37

    def run(arr, kind=0, sdt=0, blocks=blocks, rows=2, waves=4):
        return L.bp_skinny_group_run(kind, sdt, ctypes.addressof(arr), 0x5000, 0x6000, len(arr), blocks, rows, waves,
                                     None)

    assert run(arr, rows=3) == -2                                # no compiled kernel
    assert run(arr, blocks=36) == -1                             # blocks must match the plan
    arr[1].block0 = 31                                           # a stale plan
    assert run(arr) == -1
    arr[1].block0 = 32
    assert run(arr, rows=4) == -1                                # planned for 2 rows per workgroup
    int8 = _group_items([(64, 1024)], kind=1)
    assert plan(int8, kind=1) == 32
    assert run(int8, kind=1, sdt=3, blocks=32) == -1              # int8 scale dtype must be bf16 / fp16 / fp32
    empty = _group_items([(0, 512)])
    assert plan(empty) == 0
    assert run(empty, blocks=0) == 0                             # nothing to launch


# ---- the one-launch linear chain (bp_chain_*) ---------------------------------------------------------------------


def test_chain_item_layout_matches_the_header():
    from byteprof_amd.optim.linear_chain import BpChainItem

    text = HEADER.read_text()
    body = text[text.index("typedef struct BpChainItem"):text.index("} BpChainItem;")]
    fields = re.findall(r"\b(\w+);", body)
    assert [f[0] for f in BpChainItem._fields_] == fields
    assert ctypes.sizeof(BpChainItem) == 88


def _chain_item(**kw):
    from byteprof_amd.optim.linear_chain import BpChainItem

    it = BpChainItem()
    it.x, it.w, it.n, it.K, it.stage, it.dep_stage = 0x1000, 0x2000, 64, 2048, 0, -1
    for key, v in kw.items():
        setattr(it, key, v)
    return it


def _chain_plan(L, *items, rb=2, waves=8, kind=0, lut=None):
    from byteprof_amd.optim.linear_chain import BpChainItem

    arr = (BpChainItem * len(items))(*items)
    rc = L.bp_chain_plan(arr, len(items), kind, rb, waves, lut, len(lut) if lut is not None else 0)
    return rc, arr


def test_chain_plan_rejects_bad_items(L):
    assert _chain_plan(L, _chain_item())[0] == 4
    assert _chain_plan(L, _chain_item(K=1000))[0] == -1                    # K not a multiple of the segment
    assert _chain_plan(L, _chain_item(K=1024 + 64), kind=1)[0] == -1       # int8 segment is 128 elements
    assert _chain_plan(L, _chain_item(K=16384))[0] == -1                   # K above the LDS stage
    assert _chain_plan(L, _chain_item(tag_in=0x1000))[0] == -1             # two input sources
    assert _chain_plan(L, _chain_item(x=None))[0] == -1                    # no input source
    assert _chain_plan(L, _chain_item(w=0x2004))[0] == -1                  # weights not 16-byte aligned
    assert _chain_plan(L, _chain_item(x=0x1004))[0] == -1                  # external input not 8-byte aligned
    assert _chain_plan(L, _chain_item(), rb=3)[0] == -1                    # rb not 0, 1, 2, 4
    assert _chain_plan(L, _chain_item(), waves=16)[0] == -1                # waves not 2, 4, 8
    assert _chain_plan(L, _chain_item(stage=1), _chain_item(stage=0))[0] == -1          # stages out of order
    dep = dict(x=None, tag_in=0x1000, stage=1)
    assert _chain_plan(L, _chain_item(), _chain_item(dep_stage=1, **dep))[0] == -1      # depends on itself
    assert _chain_plan(L, _chain_item(stage=2), _chain_item(dep_stage=1, x=None, tag_in=0x1000, stage=3))[0] == -1
    assert _chain_plan(L, _chain_item(), _chain_item(x=None, tag_in=0x1004, stage=1, dep_stage=0))[0] == -1
    rc, arr = _chain_plan(L, _chain_item(n=100), _chain_item(n=64, stage=1), _chain_item(dep_stage=0, **dep))
    assert rc == 7 + 4 + 4 and arr[2].dep_wgs == 7 and arr[0].dep_wgs == 0
    p = ctypes.c_void_p(16)
    assert L.bp_chain_run(0, 0, None, None, 1, 1, 8, p, 0, None) == -1
    assert L.bp_chain_run(0, 0, p, p, 1, 1, 8, None, 1, None) == -3       # no scratch
    assert L.bp_chain_run(0, 0, p, p, 1, 1, 3, p, 1, None) == -2          # no kernel for 3 waves
    assert L.bp_chain_run(1, 9, p, p, 1, 1, 8, p, 1, None) == -1          # bad scale dtype


@pytest.mark.parametrize("waves", [2, 4, 8])
def test_chain_plan_sizes_tiles_to_the_slots_in_flight(L, waves):
    """rb = 0: per item, 4 blocks when a wave holds at most 4 segments, 2 up to 8, else 1 (16 in flight)."""
    for kind, seg in ((0, 64), (1, 128)):
        for k in (128, 1024, 2048, 4096, 8192):
            per_wave = -(-(k // seg) // waves)
            want = 4 if per_wave <= 4 else 2 if per_wave <= 8 else 1
            rc, arr = _chain_plan(L, _chain_item(K=k, n=1000), rb=0, waves=waves, kind=kind)
            assert arr[0].rb == want and rc == -(-1000 // (8 * want)), (kind, k, waves)


@pytest.mark.parametrize("rb", [1, 2, 4])
def test_chain_plan_places_items_in_order_with_a_lookup_table(L, rb):
    """first_wg is the running sum of ceil(n / 8 rb); lut[c] is the item holding workgroup 256 c."""
    ns = [1, 300, 5000, 8, 17, 100352, 9, 2048]
    items = [_chain_item(n=n, stage=i) for i, n in enumerate(ns)]
    total, arr = _chain_plan(L, *items, rb=rb)
    per = [-(-n // (8 * rb)) for n in ns]
    assert total == sum(per) and all(it.rb == rb for it in arr)
    starts = [sum(per[:i]) for i in range(len(ns))]
    assert [it.first_wg for it in arr] == starts
    lut = (ctypes.c_int32 * (-(-total // 256)))()
    assert _chain_plan(L, *items, rb=rb, lut=lut)[0] == total
    for c, v in enumerate(lut):
        owner = max(i for i in range(len(ns)) if starts[i] <= 256 * c)
        assert v == owner, (c, v, owner)
    short = (ctypes.c_int32 * (len(lut) - 1))()
    assert _chain_plan(L, *items, rb=rb, lut=short)[0] == -1


def test_linear_chain_builds_on_host_tensors():
    """The stage list of a decode step (CPU tensors: nothing is launched) plans into items with the right inputs,
    tagged outputs only for the stages that are read, and wait counts equal to the producer's workgroups."""
    import torch

    from byteprof_amd import decode_set as D
    from byteprof_amd.optim.linear_chain import BpChainItem, LinearChain

    weights = {name: (torch.zeros(n, k, dtype=torch.bfloat16),) for name, n, k in D.shapes()}
    for dep in (True, False):
        stages = D.chain_stages(weights, dependent=dep, device="cpu")
        ch = LinearChain(stages, rb=0, waves=8)
        assert ch.dependent == dep and ch.n_items == 113
        items = (BpChainItem * ch.n_items).from_buffer_copy(ch.items.numpy().tobytes())
        rbs = {k: 4 if k == 2048 else 1 for _, _, k in D.shapes()}  # 4 segments per wave at K = 2048, 16 at 8192
        assert [it.rb for it in items] == [rbs[k] for _, _, k in D.shapes()]
        assert ch.total_wgs == sum(-(-n // (8 * rbs[k])) for _, n, k in D.shapes())
        assert sorted(ch.tagged) == (list(range(64)) if dep else [])
        for it in items:
            st = stages[it.stage]
            if dep and it.stage > 0:
                d, start = st.src
                assert it.x is None and it.dep_stage == d and it.dep_wgs == ch.stage_wgs[d]
                assert it.tag_in == ch.tagged[d].data_ptr() + 4 * start
                assert it.flags == 1
            else:
                assert it.tag_in is None and it.x == st.src.data_ptr() and it.dep_stage == -1
            assert (it.tag_out is not None) == (it.stage in ch.tagged)
