"""Skinny weight-only matmul y[M, N] = x[M, K] @ W[N, K]^T on gfx950 (MI355X), through libbyteprof_amd.so.

Drop-in for byteprof/optim/skinny.py: same names (`skinny_mm`, `get_cfg`, `_bm`, `dequantize`, `MAX_M`, `GROUP`,
`quantize_int4`, `pack_int4`, `unpack_int4`), same argument meaning, same ValueError validation (skinny.py:136-166).
bf16 activations, fp32 accumulation, bf16 output; weights bf16 [N, K], int8 [N, K] with one scale per output row
(bf16, fp16 or fp32), or int4 group-128 in the reference's tile-major format.

bf16 and int8 run on one matrix-core kernel family for every row count (csrc/skinny_mf.h): one launch takes up to
MAX_M = 64 activation rows and streams every weight byte once; the K order of every sum depends only on the shape's
(waves, split), never on M, so output row i is bitwise the same whether it is computed alone or with up to 63 other
rows (the reference's row-independence contract, test_skinny.py:110-120, here over M = 1..64). int4 runs on
skinny_int4.hip (VALU dot products whose order also ignores M).

`cfg` is (rows, waves, split) for the bf16 / int8 kernel (rows: weight rows per workgroup, a multiple of 8;
waves: wavefronts sharing a workgroup's K range; split: K ranges in separate workgroups, added in fixed order) or
the reference's (BN, BK, num_warps, num_stages[, split]), mapped to (BN, num_warps, split). Differences from the
reference forced by raw-pointer kernels: x must be bfloat16 and on the GPU, w, scale and out contiguous.
"""

from __future__ import annotations

import ctypes

import functools
import json
from pathlib import Path

import torch

from .. import _lib

GROUP = 128
MAX_M = 64  # activation rows per launch; more rows are processed in chunks of MAX_M (skinny.py:32)
ROWS_PER_LAUNCH = MAX_M

_KIND_CODE = {"bf16": 0, "int8": 1}
XS_STAGE, XS_GENERAL = 1, 2  # BP_XS_STAGE, BP_XS_GENERAL: activations staged in LDS; the general segment loop
XS_ROWS2, XS_ROWS4 = 4, 8     # BP_XS_ROWS2 / 4: with XS_STAGE at 9..16 rows, 2 / 4 row groups over one staged copy
XS_ROWS = XS_ROWS2 | XS_ROWS4
_RB_MENU = (1, 2, 4)        # 8-row weight blocks per workgroup
_WAVES_MENU = (1, 2, 4, 8)
_BUCKETS = (1, 8, 16, 32, 64)  # row buckets of the tuned plans (8-row activation blocks per launch: 1, 1, 2, 4, 8)

# Tuned (waves, split) per (kind, N, K) -- one K order for every row count -- and weight blocks per workgroup per
# activation-row bucket; written by byteprof_amd.tune.
_CFG_FILE = Path(__file__).with_name("skinny_cfg.json")
_TABLE: dict[tuple[str, int, int], dict] = {}
if _CFG_FILE.exists():
    for _key, _v in json.loads(_CFG_FILE.read_text(encoding="utf-8")).items():
        if _key.startswith("_"):
            continue
        _kind, _n, _k = _key.split("|")
        _TABLE[(_kind, int(_n), int(_k))] = _v


def _bm(m: int) -> int:
    """The reference's row bucket of a launch (skinny.py:108-109): 16, 32 or 64."""
    return 16 if m <= 16 else 32 if m <= 32 else 64


def _bucket(m: int) -> int:
    """Row bucket of a launch's tuned plan: 1 (the decode step), else M rounded up to 8, 16, 32 or 64. The plan
    (weight blocks per workgroup, activation staging) may differ per bucket; the K order may not."""
    for b in _BUCKETS:
        if m <= b:
            return b
    return MAX_M


def k_segment(kind: str) -> int:
    """K elements of one weight row that one load instruction of the kernel covers (64 bf16, 128 int8)."""
    return 64 if kind == "bf16" else 128


def _default_waves(kind: str, k: int) -> int:
    nseg = -(-k // k_segment(kind))
    waves = 1
    while waves * 2 <= 8 and nseg // (waves * 2) >= 4:  # at least 4 segments per wave
        waves *= 2
    return waves


def _default_rb(n: int, bucket: int) -> int:
    blocks = -(-n // 8)
    if bucket > 16:
        return 1
    return 2 if blocks >= 2048 else 1


def _default_split(kind: str, n: int, k: int, waves: int) -> int:
    blocks = -(-n // 8)
    nseg = -(-k // k_segment(kind))
    split = 1
    while blocks * split < 256 and nseg // (waves * split * 2) >= 2:
        split *= 2
    return split


def get_cfg(kind: str, n: int, k: int, bm: int) -> tuple[int, int, int]:
    """(rows, waves, split) of a bf16 / int8 launch of `bm` activation rows (the bucket's upper bound): the tuned
    table first, then a heuristic. waves and split (the K order) depend on the shape only."""
    rb, waves, split, _ = _table_plan(kind, n, k, bm)
    return 8 * rb, waves, split


def _table_plan(kind: str, n: int, k: int, m: int, pro: bool = False) -> tuple[int, int, int, int]:
    """(weight blocks per workgroup, waves, split, xstage flags) from the table, else the heuristic. pro: a launch
    with a norm prologue, whose weight blocks per workgroup the table may tune apart (rb_pro; same K order)."""
    bucket = _bucket(m)
    entry = _TABLE.get((kind, n, k))
    if entry is not None:
        rb = int(entry.get("rb", {}).get(str(bucket), _default_rb(n, bucket)))
        if pro:
            rb = int(entry.get("rb_pro", {}).get(str(bucket), rb))
        xs = int(entry.get("xs", {}).get(str(bucket), 0))
        return rb, int(entry["waves"]), int(entry.get("split", 1)), xs
    waves = _default_waves(kind, k)
    return _default_rb(n, bucket), waves, _default_split(kind, n, k, waves), int(n >= 16384)


def _resolve(kind: str, n: int, k: int, m: int, cfg, pro: bool = False) -> tuple[int, int, int, int]:
    """(weight blocks per workgroup, waves, split, xstage flags) of a launch from a user / table configuration,
    mapped onto the compiled menu (largest supported value at or below the request); pro: a norm-prologue launch."""
    xs = 0
    if cfg is None:
        rb, waves, split, xs = _table_plan(kind, n, k, m, pro)
        rows = 8 * rb
    elif len(cfg) == 3:
        rows, waves, split = (int(c) for c in cfg)
    elif len(cfg) in (4, 5):  # the reference's (BN, BK, num_warps, num_stages[, split])
        rows, waves, split = int(cfg[0]), int(cfg[2]), int(cfg[4]) if len(cfg) == 5 else 1
    else:
        raise ValueError(f"cfg must be (rows, waves, split) or (BN, BK, warps, stages[, split]), got {cfg!r}")
    rb = max(r for r in _RB_MENU if r <= max(rows // 8, 1))
    waves = max(w for w in _WAVES_MENU if w <= max(waves, 1))
    split = max(1, min(int(split), -(-k // k_segment(kind))))
    if xs & XS_STAGE and (m > 16 or _stage_bytes(kind, m, k, split, xs) < 0):
        xs &= ~(XS_STAGE | XS_ROWS)
    if not xs & XS_STAGE or not 8 < m <= 16 or not _supported(kind, m, rb, waves, xs & (XS_STAGE | XS_ROWS)):
        xs &= ~XS_ROWS  # row groups: staged 9..16-row launches of a compiled (rb, waves)
    while rb > 1 and not _supported(kind, m, rb, waves, xs & (XS_STAGE | XS_ROWS)):
        rb //= 2
    if not _supported(kind, m, rb, waves, xs & (XS_STAGE | XS_ROWS)):
        raise ValueError(f"no compiled kernel for {kind} at {m} rows, {8 * rb} weight rows, {waves} waves")
    return rb, waves, split, xs


def segments_per_wave(kind: str, k: int, waves: int, split: int, xs: int = 0) -> int:
    """K segments every wave of a launch handles when the launch runs the straight-line kernel of that count (4, 8
    or 16: the split ranges and the waves divide K's segments evenly, and XS_GENERAL is not set), else 0."""
    seg = k_segment(kind)
    if k % seg or xs & XS_GENERAL:
        return 0
    nseg = k // seg
    if nseg % split or (nseg // split) % waves:
        return 0
    n = nseg // split // waves
    return n if n in (4, 8, 16) else 0


def kernel_name(kind: str, n: int, k: int, m: int, cfg=None) -> str:
    """Name of the kernel instantiation a skinny_mm launch of m rows runs, as the profiler reports it (template
    arguments: kind, activation blocks, weight blocks, waves, vector loads, epilogue, staged activations, prologue,
    segments per wave, row groups)."""
    rb, waves, split, xs = _resolve(kind, n, k, m, cfg)
    mb = 1 if m <= 8 else 2 if m <= 16 else 4 if m <= 32 else 8
    wr = 4 if xs & XS_ROWS4 else 2 if xs & XS_ROWS2 else 1
    nseg = segments_per_wave(kind, k, waves, split, xs)
    if wr > 1 and nseg == 16:
        nseg = 0  # the row-group kernels run the general loop there
    return (f"skinny_mf_kernel<{_KIND_CODE[kind]}, {mb}, {rb}, {waves}, true, 0, "
            f"{'true' if xs & XS_STAGE else 'false'}, false, {nseg}, {wr}>")


@functools.lru_cache(maxsize=None)
def _supported(kind: str, m: int, rb: int, waves: int, xs: int = 0) -> bool:
    return bool(_lib.lib().bp_skinny_mf_supported(_KIND_CODE[kind], m, rb, waves, xs))


@functools.lru_cache(maxsize=None)
def _stage_bytes(kind: str, m: int, k: int, split: int, xs: int = 0) -> int:
    if xs & XS_ROWS:
        return int(_lib.lib().bp_skinny_mf_stage_bytes_rows(_KIND_CODE[kind], m, k, split, xs))
    return int(_lib.lib().bp_skinny_mf_stage_bytes(_KIND_CODE[kind], m, k, split))


def _launch(kind: str, x: torch.Tensor, w: torch.Tensor, scale, y: torch.Tensor, cfg=None) -> None:
    m, k = x.shape
    n = w.shape[0]
    rb, waves, split, xs = _resolve(kind, n, k, m, cfg)
    L = _lib.lib()
    ws = None
    ws_bytes = 0
    if split > 1:
        ws_bytes = L.bp_skinny_workspace_bytes(m, n, split)
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=x.device)
    sc, sdt = (scale.data_ptr(), _lib.TORCH_DT[scale.dtype]) if kind == "int8" else (None, 0)
    rc = L.bp_skinny_mf(_KIND_CODE[kind], x.data_ptr(), w.data_ptr(), sc, sdt, y.data_ptr(), m, n, k, rb, waves,
                        split, xs, _lib.ptr(ws), ws_bytes, _lib.stream_ptr(x.device))
    _lib.check(rc, f"bp_skinny_mf ({kind})")


class BpPrologue(ctypes.Structure):
    """Mirror of `BpPrologue` in include/byteprof_amd.h (40 bytes)."""

    _fields_ = [("kind", ctypes.c_int32), ("eps", ctypes.c_float), ("gamma", ctypes.c_void_p),
                ("residual", ctypes.c_void_p), ("xout", ctypes.c_void_p), ("gamma2", ctypes.c_void_p)]


PRO_UNIT_RMS, PRO_NORM = 1, 2  # BP_PRO_UNIT_RMS, BP_PRO_NORM


def prologue_mm(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor | None, out: torch.Tensor, pro: int,
                gamma: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                xout: torch.Tensor | None = None, eps: float = 0.0, silu: bool = False, cfg=None,
                gamma2: torch.Tensor | None = None, zero: torch.Tensor | None = None) -> None:
    """out = (transform of x) . W^T in one launch (bp_skinny_mf_pro; int4 weights with zero: bp_skinny_int4_pro):
    pro PRO_UNIT_RMS renormalises each row of x to unit RMS, PRO_NORM takes bf16(residual + bf16(gamma *
    rmsnorm(x))) (the decode norm kernel's arithmetic), then with gamma2 the plain norm of that with weight gamma2;
    xout, when given, receives the rows before the second norm. silu: w is the interleaved gate|up weight [2 F, K]
    and out [M, F] the SiLU product. The shape's plan must have split 1 (rows x K of x are staged in LDS; M <= 16;
    int4: M <= 8 and (2 M + 2) K bf16 within 64 KiB, bf16 scales)."""
    m, k = x.shape
    if w.dtype == torch.uint8:
        kind = "int4"
        if zero is None or scale is None:
            raise ValueError("int4 weights need scale and zero")
        tile = int(w.shape[2])
        n = scale.shape[1] // (2 if silu else 1)
        waves, split = int4_cfg(scale.shape[1], k, tile, cfg)
        split = min(split, k // GROUP)
    else:
        n = w.shape[0] // (2 if silu else 1)
        kind = "bf16" if scale is None else "int8"
        rb, waves, split, _ = _resolve(kind, w.shape[0], k, m, cfg, pro=True)
    if split != 1:
        raise ValueError(f"a prologue needs whole rows per workgroup: the {w.shape[0]}x{k} plan splits K {split} ways")
    for t in (x, w, out, gamma, residual, xout, gamma2):
        if t is not None and not t.is_contiguous():
            raise ValueError("prologue_mm operands must be contiguous")
    wk = w.shape[1] * GROUP if kind == "int4" else w.shape[1]
    if x.dtype != torch.bfloat16 or wk != k:
        raise ValueError(f"prologue_mm: x must be bf16 [M, {wk}]")
    if out.shape != (m, n) or out.dtype != torch.bfloat16:
        raise ValueError(f"prologue_mm: out must be a bf16 [{m}, {n}] tensor")
    for t, rows in ((gamma, None), (gamma2, None), (residual, m), (xout, m)):
        if t is not None and (t.dtype != torch.bfloat16 or t.numel() != (k if rows is None else rows * k)):
            raise ValueError("prologue_mm: gamma / gamma2 must be bf16 [K], residual / xout bf16 [M, K]")
    if xout is not None:
        # one workgroup writes xout while the others still read x and the residual rows
        rows = 2 * m * k
        for t in (x, residual):
            if t is not None and xout.data_ptr() < t.data_ptr() + rows and t.data_ptr() < xout.data_ptr() + rows:
                raise ValueError("prologue_mm: xout must not overlap x or residual")
    p = BpPrologue(pro, eps, _lib.ptr(gamma), _lib.ptr(residual), _lib.ptr(xout), _lib.ptr(gamma2))
    sc, sdt = (scale.data_ptr(), _lib.TORCH_DT[scale.dtype]) if scale is not None else (None, 0)
    L = _lib.lib()
    if kind == "int4":
        rc = L.bp_skinny_int4_pro(x.data_ptr(), w.data_ptr(), sc, sdt, zero.data_ptr(), out.data_ptr(), m, n, k, tile,
                                  waves, int(silu), ctypes.byref(p), _lib.stream_ptr(x.device))
        _lib.check(rc, "bp_skinny_int4_pro")
        return
    rc = L.bp_skinny_mf_pro(_KIND_CODE[kind], x.data_ptr(), w.data_ptr(), sc, sdt, out.data_ptr(), m, n, k, rb, waves,
                            int(silu), ctypes.byref(p), _lib.stream_ptr(x.device))
    _lib.check(rc, "bp_skinny_mf_pro")


def _check_device(x: torch.Tensor, *others: torch.Tensor | None) -> None:
    if not x.is_cuda:
        raise ValueError("x must be on a GPU (the skinny kernels have no CPU path)")
    for t in others:
        if t is not None and t.device != x.device:
            raise ValueError(f"all tensors must be on {x.device}, got {t.device}")


def skinny_mm(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor | None = None,
              zero: torch.Tensor | None = None, out: torch.Tensor | None = None,
              cfg: tuple[int, ...] | None = None) -> torch.Tensor:
    """x: [M, K] bf16 (contiguous); w: bf16 [N, K] | int8 [N, K] + scale [N] | int4 tile-major uint8 + scale,
    zero [K/128, N]. Returns y [M, N] in x.dtype (written into `out` when given).

    Validation and empty-shape behaviour follow byteprof/optim/skinny.py:136-166."""
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous [M, K] tensor")
    m, k = x.shape
    if w.dtype == torch.bfloat16:
        kind, n = "bf16", w.shape[0]
        if w.shape[1] != k:
            raise ValueError("K mismatch")
    elif w.dtype == torch.int8:
        kind, n = "int8", w.shape[0]
        if scale is None or w.shape[1] != k:
            raise ValueError("int8 needs scale [N] and K to match")
        if scale.dim() != 1 or scale.shape[0] != n or not scale.is_contiguous() or scale.dtype not in (
                torch.bfloat16, torch.float16, torch.float32):
            raise ValueError("int8 scale must be a contiguous [N] bf16 / fp16 / fp32 tensor")
    elif w.dtype == torch.uint8:
        if scale is None or zero is None or w.dim() != 4 or k % GROUP or w.shape[1] * GROUP != k or \
                scale.shape[0] != w.shape[1]:
            raise ValueError("int4 needs packed [N/R, K/128, R, 64], scale/zero [K/128, N] and K % 128 == 0")
        kind, n = "int4", scale.shape[1]
        if scale.dim() != 2 or zero.shape != scale.shape or zero.dtype != torch.float16 or w.shape[3] != 64 or \
                w.shape[0] * w.shape[2] < n or scale.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise ValueError("int4 needs scale [K/128, N] (bf16 / fp16 / fp32) and zero [K/128, N] fp16 matching the "
                             "packed weights")
    else:
        raise ValueError(f"unsupported weight dtype {w.dtype}")
    if kind != "int4" and (w.dim() != 2 or not w.is_contiguous()):
        raise ValueError("w must be a contiguous [N, K] tensor")
    if kind == "int4" and not (w.is_contiguous() and scale.is_contiguous() and zero.is_contiguous()):
        raise ValueError("int4 packed weights, scale and zero must be contiguous")
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bfloat16")
    _check_device(x, w, scale, zero, out)
    if out is not None:
        if out.shape != (m, n) or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous [{m}, {n}] {x.dtype} tensor")
        y = out
    else:
        y = torch.empty(m, n, dtype=x.dtype, device=x.device)
    if m == 0 or n == 0 or k == 0:
        if k == 0:
            y.zero_()
        return y
    if kind == "int4":
        for r0 in range(0, m, INT4_ROWS_PER_LAUNCH):
            _launch_int4(x[r0:r0 + INT4_ROWS_PER_LAUNCH], w, scale, zero, y[r0:r0 + INT4_ROWS_PER_LAUNCH], cfg)
    else:
        for r0 in range(0, m, MAX_M):
            _launch(kind, x[r0:r0 + MAX_M], w, scale, y[r0:r0 + MAX_M], cfg)
    return y


INT4_ROWS_PER_LAUNCH = 16  # activation rows per launch of the int4 kernel


INT4_TILES = (16, 32, 64)  # tile rows of the int4 matrix-core kernel on gfx950


def int4_tile_rows(n: int, k: int) -> int:
    """Tile rows to pack an int4 weight [N, K] with: the tuned table entry 'int4|N|K' (the tile rows whose plan is
    fastest at M = 1), else by N: more rows per workgroup for larger N (one wave per 64-row tile streams the LM head
    fastest; 16-row tiles keep small matrices on enough workgroups)."""
    entry = _TABLE.get(("int4", n, k))
    if entry is not None and int(entry.get("tile_rows", 32)) in INT4_TILES:
        return int(entry.get("tile_rows", 32))
    return 64 if n >= 32768 else 16 if n <= 4096 else 32


def int4_cfg(n: int, k: int, tile_rows: int, cfg=None) -> tuple[int, int]:
    """(waves, split) of an int4 launch on weights packed in tiles of tile_rows: the tuned table entry 'int4|N|K'
    for those tile rows, else a heuristic; a user cfg is (waves, split) or the reference's (BN, BK, warps,
    stages[, split])."""
    if cfg is not None:
        if len(cfg) == 2:
            waves, split = int(cfg[0]), int(cfg[1])
        elif len(cfg) in (4, 5):
            waves, split = int(cfg[2]), int(cfg[4]) if len(cfg) == 5 else 1
        else:
            raise ValueError(f"int4 cfg must be (waves, split) or (BN, BK, warps, stages[, split]), got {cfg!r}")
    else:
        entry = _TABLE.get(("int4", n, k)) or {}
        plan = entry.get("tiles", {}).get(str(tile_rows))
        if plan is None and entry and int(entry.get("tile_rows", 32)) == tile_rows:
            plan = entry
        if plan is not None:
            waves, split = int(plan["waves"]), int(plan.get("split", 1))
        else:
            groups = k // GROUP
            waves = 1 if tile_rows == 64 else 4 if tile_rows == 16 else 8
            while waves > 1 and waves > groups:
                waves //= 2
            split = 1
    waves = max(w for w in (1, 2, 4, 8) if w <= max(waves, 1))
    return waves, max(1, split)


def _launch_int4(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, y: torch.Tensor,
                 cfg=None) -> None:
    m, k = x.shape
    n = scale.shape[1]
    tile_rows = int(w.shape[2])
    if tile_rows not in (16, 32, 64):
        raise ValueError(f"int4 tile rows must be 16, 32 or 64 on gfx950, got {tile_rows}")
    waves, split = int4_cfg(n, k, tile_rows, cfg)
    split = min(split, k // GROUP)
    if x.data_ptr() % 16:
        x = x.clone()
    L = _lib.lib()
    ws = None
    ws_bytes = 0
    if split > 1:
        ws_bytes = L.bp_skinny_workspace_bytes(m, n, split)
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=x.device)
    rc = L.bp_skinny_int4(x.data_ptr(), w.data_ptr(), scale.data_ptr(), _lib.TORCH_DT[scale.dtype], zero.data_ptr(),
                          y.data_ptr(), m, n, k, tile_rows, waves, split, _lib.ptr(ws), ws_bytes,
                          _lib.stream_ptr(x.device))
    _lib.check(rc, "bp_skinny_int4")


def quantize_int4(w: torch.Tensor, tile_rows: int = 32) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Asymmetric group-128 int4 of w [N, K] (byteprof/optim/skinny.py:172-185): per row and group of 128 inputs,
    scale = max((max - min) / 15, 1e-6) stored in w.dtype, zero = -min / scale stored in fp16, code =
    round_half_even(w / scale + zero) clamped to 0..15 (fp32 arithmetic). Returns (packed [ceil(N/R), K/128, R, 64]
    uint8, scale [K/128, N] w.dtype, zero [K/128, N] fp16)."""
    n, k = w.shape
    if k % GROUP:
        raise ValueError("int4 needs K % 128 == 0")
    groups = w.float().reshape(n, k // GROUP, GROUP)
    lo, hi = groups.amin(dim=-1), groups.amax(dim=-1)
    scale = ((hi - lo) / 15.0).clamp_min(1e-6).to(w.dtype)
    zero = (-lo / scale.float()).to(torch.float16)
    codes = torch.round(groups / scale.float().unsqueeze(-1) + zero.float().unsqueeze(-1)).clamp_(0, 15)
    return pack_int4(codes.to(torch.uint8).reshape(n, k), tile_rows), scale.t().contiguous(), zero.t().contiguous()


def pack_int4(codes: torch.Tensor, tile_rows: int = 32) -> torch.Tensor:
    """Codes 0..15 [N, K] -> the tile-major layout [ceil(N/R), K/128, R, 64] (byteprof/optim/skinny.py:188-198):
    within a row's group of 128, byte j = code j | code (j + 64) << 4; the R rows of a tile and group are one
    contiguous R x 64-byte block; padding rows are zero."""
    n, k = codes.shape
    tiles = -(-n // tile_rows)
    full = codes.new_zeros(tiles * tile_rows, k)
    full[:n] = codes
    g = full.reshape(tiles, tile_rows, k // GROUP, 2, GROUP // 2)
    return (g[:, :, :, 0] | (g[:, :, :, 1] << 4)).permute(0, 2, 1, 3).contiguous()


def unpack_int4(packed: torch.Tensor, n: int) -> torch.Tensor:
    """Inverse of pack_int4: codes [N, K] (byteprof/optim/skinny.py:201-206)."""
    tiles, groups, rows, _ = packed.shape
    p = packed.permute(0, 2, 1, 3)
    return torch.stack([p & 0xF, p >> 4], dim=3).reshape(tiles * rows, groups * GROUP)[:n]


def dequantize(kind: str, w: torch.Tensor, scale=None, zero=None) -> torch.Tensor:
    """fp32 weights [N, K] of a stored format (byteprof/optim/skinny.py:209-217)."""
    if kind == "bf16":
        return w.float()
    if kind == "int8":
        return w.float() * scale.float()[:, None]
    groups, n = scale.shape
    codes = unpack_int4(w, n).float().reshape(n, groups, GROUP) - zero.float().t().unsqueeze(-1)
    return (codes * scale.float().t().unsqueeze(-1)).reshape(n, groups * GROUP)
