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
    for required in ("bp_skinny_mf", "bp_skinny_mf_partials", "bp_skinny_mf_silu", "bp_skinny_mf_supported",
                     "bp_splitk_reduce", "bp_mlstm_multistep", "bp_skinny_workspace_bytes", "bp_version",
                     "bp_status_string", "bp_chain_plan", "bp_chain_run", "bp_chain_scratch_bytes",
                     "bp_chain_supported", "bp_skinny_int4"):
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
    # every (rows per launch, weight blocks, waves) the planner may pick is compiled, for both kinds
    for kind in (0, 1):
        for m in (1, 2, 5, 8, 9, 16, 17, 33, 64):
            for waves in (1, 2, 4, 8):
                assert L.bp_skinny_mf_supported(kind, m, 1, waves, 0), (kind, m, waves)
        for rb in (1, 2, 4):
            assert L.bp_skinny_mf_supported(kind, 1, rb, 4, 0)
    assert not L.bp_skinny_mf_supported(0, 1, 3, 4, 0)   # rb is 1, 2 or 4
    assert not L.bp_skinny_mf_supported(0, 65, 1, 4, 0)  # at most 64 rows per launch
    assert not L.bp_skinny_mf_supported(2, 1, 1, 4, 0)   # kinds are 0 (bf16) and 1 (int8)
    assert L.bp_skinny_mf_k_segment(0) == 64 and L.bp_skinny_mf_k_segment(1) == 128


def test_invalid_arguments_are_rejected_before_any_launch(L):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below returns before enqueueing anything
    mf = lambda kind, x, w, sc, sdt, m, n, k, rb=1, waves=4, split=1, ws=None, wsb=0: L.bp_skinny_mf(  # noqa: E731
        kind, x, w, sc, sdt, p, m, n, k, rb, waves, split, 0, ws, wsb, None)
    assert mf(0, None, p, None, 0, 1, 1, 64) == -1          # null x
    assert mf(0, p, p, None, 0, -1, 1, 64) == -1            # negative M
    assert mf(0, p, p, None, 0, 65, 1, 64) == -1            # more than 64 rows
    assert mf(0, p, p, None, 0, 0, 5, 64) == 0              # M = 0: no-op
    assert mf(0, p, p, None, 0, 3, 0, 64) == 0              # N = 0: no-op
    assert mf(0, p, p, None, 0, 1, 8, 1024, rb=3) == -2     # rb not in the menu
    assert mf(0, p, p, None, 0, 1, 8, 4096, split=2) == -3  # split without workspace
    assert mf(1, p, p, None, 0, 1, 8, 128) == -1            # int8 without scale
    assert mf(1, p, p, p, 7, 1, 8, 128) == -1               # bad scale dtype
    assert L.bp_splitk_reduce(None, p, None, 0, 2, 2, 2, None) == -1
    # mLSTM: DQ not a multiple of 64, bad value block, DV not a multiple of it
    args = [p] * 11
    assert L.bp_mlstm_multistep(*args, 4, 2, 48, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == -2
    assert L.bp_mlstm_multistep(*args, 4, 2, 64, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 5, None) == -2
    assert L.bp_mlstm_multistep(*args, 4, 2, 64, 12, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == -2
    assert L.bp_mlstm_multistep(*args, 4, 0, 64, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == 0  # NH = 0: no-op
    # DQ whose workgroup would not be whole waves (320 -> 160 threads, 448 -> 224), or beyond 512
    for dq in (320, 448, 576):
        assert L.bp_mlstm_multistep(*args, 4, 2, dq, 16, 1, 1, 1, 1, 0, 2, 0.1, 1e-6, 8, None) == -2, dq
        assert L.bp_mlstm_lazy_commit(*[p] * 10, 4, 2, dq, 16, 1, 1, 1, 0, 2, 8, None) == -2, dq
    assert L.bp_mlstm_step(*[p] * 12, 2, 320, 16, 0, 2, 0.1, 1e-6, 8, None) == -2
    assert L.bp_mlstm_step(*[p] * 9, None, p, p, 2, 64, 16, 0, 2, 0.1, 1e-6, 8, None) == -1  # no new state
    # the argmax's partial words are 64-bit: its scratch must be 8-byte aligned
    odd = ctypes.c_void_p(20)
    assert L.bp_decode_argmax_next(p, 100, p, p, odd, None) == -1
    assert L.bp_decode_argmax_rows(p, 100, 2, p, odd, None) == -1
    assert L.bp_decode_argmax_scratch_bytes() % 8 == 0 and L.bp_decode_argmax_rows_scratch_bytes(3) % 8 == 0
    # the verify attention's q|k|v rows must fit one buffer resource (2^31 bytes): 16 rows x 3 x 2^25 x 2 bytes
    ra = lambda heads, rows: L.bp_decode_rope_attention_rows(p, p, p, p, p, p, p, p, heads, 128, rows, 64,  # noqa: E731
                                                             1e-6, 0.1, None)
    assert ra(1 << 18, 16) == -2
    assert ra(0, 16) == -1


def test_argmax_scratch_holds_an_error_word_per_row(L):
    """Per row: 64 partial words (64-bit), the generation, the counter, the error word and a pad word, so every
    row's partials stay 8-byte aligned; the host reads the error word at the place the header names."""
    from byteprof_amd.optim import olmo

    text = HEADER.read_text()
    row_words = int(re.search(r"#define BP_ARGMAX_ROW_WORDS (\d+)", text).group(1))
    error_word = int(re.search(r"#define BP_ARGMAX_ERROR_WORD (\d+)", text).group(1))
    assert (row_words, error_word) == (olmo.ARGMAX_ROW_WORDS, olmo.ARGMAX_ERROR_WORD) == (132, 130)
    assert L.bp_decode_argmax_scratch_bytes() == 4 * row_words
    for rows in (1, 3, 16):
        assert L.bp_decode_argmax_rows_scratch_bytes(rows) == 4 * row_words * rows
    assert L.bp_decode_argmax_rows_scratch_bytes(0) == 0


def _prologue(**kw):
    from byteprof_amd.optim.skinny import BpPrologue

    pr = BpPrologue()
    pr.kind, pr.eps, pr.gamma = 2, 1e-6, 0x100000
    for key, v in kw.items():
        setattr(pr, key, v)
    return pr


def test_prologue_refuses_an_xout_overlapping_its_inputs(L):
    """Workgroup (0, 0) writes xout while the others still read x and the residual rows: an xout whose M x K
    elements intersect either is refused before anything is enqueued."""
    x, w, y, res = 0x200000, 0x400000, 0x600000, 0x800000
    m, n, k = 2, 64, 2048
    rows = 2 * m * k
    pro = lambda pr: L.bp_skinny_mf_pro(0, x, w, None, 0, y, m, n, k, 1, 4, 0,  # noqa: E731
                                        ctypes.byref(pr), None)
    for xout in (x, x + rows - 16, x - rows + 16):  # the same rows, their last 16 bytes, their first 16 bytes
        assert pro(_prologue(xout=xout)) == -1, hex(xout)
        assert pro(_prologue(kind=1, gamma=None, xout=xout)) == -1, hex(xout)
    for xout in (res, res + rows - 16, res - rows + 16):
        assert pro(_prologue(residual=res, xout=xout)) == -1, hex(xout)


def test_int4_prologue_refusals_before_any_launch(L):
    """bp_skinny_int4_pro checks its arguments before any HIP call (the pointers are never used): no prologue, an
    unknown kind or epilogue, NORM without gamma, unaligned norm operands, gamma2 with the unit-RMS kind and an xout
    overlapping x or the residual row are invalid; nine rows, rows whose staging passes 64 KiB of LDS and K not a
    multiple of 128 are refused."""
    x, pk, sc, z, y, res = 0x200000, 0x400000, 0x600000, 0x800000, 0xa00000, 0xc00000
    n, k = 64, 2048
    call = lambda pr, m=1, k_=k, epi=0: L.bp_skinny_int4_pro(  # noqa: E731
        x, pk, sc, 0, z, y, m, n, k_, 16, 4, epi, None if pr is None else ctypes.byref(pr), None)
    assert call(None) == -1
    assert call(_prologue(), epi=2) == -1
    assert call(_prologue(kind=7)) == -1
    assert call(_prologue(gamma=None)) == -1
    assert call(_prologue(gamma=0x100008)) == -1
    assert call(_prologue(residual=res + 8)) == -1
    assert call(_prologue(kind=1, gamma=None, gamma2=0x100000)) == -1
    for xout in (x, x + 2 * k - 16, res):
        assert call(_prologue(residual=res, xout=xout)) == -1, hex(xout)
    assert call(_prologue(), m=9) == -2
    assert call(_prologue(), m=2, k_=8192) == -2  # (2 M + 2) K bf16 past 64 KiB
    assert call(_prologue(), m=7, k_=2176) == -2
    assert call(_prologue(), k_=8320) == -2
    assert call(_prologue(), k_=2000) == -1
    assert call(_prologue(), m=0) == 0  # nothing to do


def test_prologue_mm_refuses_an_overlapping_xout_on_the_host():
    import torch

    from byteprof_amd.optim import skinny as S

    x = torch.zeros(4, 2048, dtype=torch.bfloat16)
    w = torch.zeros(2048, 2048, dtype=torch.bfloat16)  # a tuned shape whose plan keeps whole rows (split 1)
    out = torch.zeros(4, 2048, dtype=torch.bfloat16)
    g = torch.ones(2048, dtype=torch.bfloat16)
    res = torch.zeros(4, 2048, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="overlap"):
        S.prologue_mm(x, w, None, out, S.PRO_NORM, gamma=g, residual=res, xout=x, eps=1e-6)
    with pytest.raises(ValueError, match="overlap"):
        S.prologue_mm(x, w, None, out, S.PRO_NORM, gamma=g, residual=res, xout=res, eps=1e-6)
    big = torch.zeros(8, 2048, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="overlap"):  # the last rows of one buffer are the first of the other
        S.prologue_mm(big[:4], w, None, out, S.PRO_UNIT_RMS, xout=big[3:7])
    # operands whose shapes do not match the launch are refused before any pointer reaches the library
    with pytest.raises(ValueError, match="out must"):
        S.prologue_mm(x, w, None, out[:3], S.PRO_NORM, gamma=g, eps=1e-6)
    with pytest.raises(ValueError, match="gamma"):
        S.prologue_mm(x, w, None, out, S.PRO_NORM, gamma=g[:1024], eps=1e-6)
    with pytest.raises(ValueError, match="residual"):
        S.prologue_mm(x, w, None, out, S.PRO_NORM, gamma=g, residual=res[:2], eps=1e-6)
    with pytest.raises(ValueError, match="x must"):
        S.prologue_mm(x[:, :1024].contiguous(), w, None, out, S.PRO_UNIT_RMS)


def test_static_scratch_entry_refuses_partials_beyond_its_array(L):
    """bp_skinny_mf_static's split-K partials live in an 8 MiB device array: a call whose split x M x N x 4
    bytes exceed it is refused before any HIP call (the pointers are never used)."""
    p = ctypes.c_void_p(16)
    assert L.bp_skinny_mf_static_bytes() == 8 << 20
    assert L.bp_skinny_mf_static(0, p, p, None, 0, p, 16, 100352 * 8, 2048, 1, 4, 2, 0, None) == -3
    assert L.bp_skinny_mf_static(1, p, p, p, 1, p, 16, 65537, 2048, 1, 4, 2, 0, None) == -3  # 8 MiB + 128 bytes
    assert L.bp_skinny_mf_static(0, p, p, None, 0, p, 1, 8, 2048, 1, 4, 0, 0, None) == -1    # split 0
    assert L.bp_skinny_mf_static(0, p, p, None, 0, p, -1, 8, 2048, 1, 4, 1, 0, None) == -1   # negative M


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
