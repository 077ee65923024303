"""Skinny weight-only matmul y[M, N] = x[M, K] @ W[N, K]^T on gfx950 (MI355X), through libbyteprof_amd.so.

Drop-in for byteprof/optim/skinny.py: same names (`skinny_mm`, `get_cfg`, `dequantize`, `MAX_M`, `GROUP`), same
argument meaning, same ValueError validation (skinny.py:136-166). bf16 activations, fp32 accumulation, bf16 output;
weights bf16 [N, K] or int8 [N, K] with one scale per output row (bf16, fp16 or fp32).

Differences from the reference, each forced by the hardware mapping or by raw-pointer kernels:
  - one launch handles up to ROWS_PER_LAUNCH = 16 activation rows (the reference: 64); larger M is chunked here,
    and `SkinnyLinear` still sends every input of 1..MAX_M rows to the kernel;
  - x must be bfloat16 and on the GPU, w and scale contiguous (the reference assumes the latter silently);
  - `cfg` is (rows, waves, split) for this kernel (rows: weight rows per workgroup; waves: wavefronts sharing the
    K range of a workgroup; split: K ranges in separate workgroups, added in fixed order). The reference's
    (BN, BK, num_warps, num_stages[, split]) tuples are accepted and mapped to (BN, num_warps, split);
  - launches of 5..16 rows (the 8- and 16-row buckets: speculative-verify widths) run on the matrix cores
    (skinny_mfma.hip) when K is a multiple of 128 (bf16) / 256 (int8), launches of 1..4 rows on the VALU dot2
    kernels; bitwise row independence (test_skinny.py:114-121) holds within each family, i.e. for M = 1..4 and for
    M = 5..16 (the reference's single M <= 16 bucket is split at the change of arithmetic unit). An explicit `cfg`
    selects the VALU kernel;
  - int4 group-128 weights (uint8 tile-major, `quantize_int4` / `pack_int4`, the reference's format byte for byte)
    run on skinny_int4.hip, whose products use the codes, zeros and activations exactly (the reference rounds
    code - zero to bf16 before its tensor-core product): closer to the dequantize-then-matmul result.
"""

from __future__ import annotations

import functools
import json
from pathlib import Path

import torch

from .. import _lib

GROUP = 128
MAX_M = 64  # rows for which SkinnyLinear uses the kernel (skinny_linear.py:60); interface parity with the reference
ROWS_PER_LAUNCH = 16  # activation rows per kernel launch on gfx950

_ROW_BUCKETS = (1, 2, 4, 8, 16)
_ROWS_MENU = (2, 4, 8, 16, 32)
_WAVES_MENU = (1, 2, 4, 8, 16)
_KIND_CODE = {"bf16": 0, "int8": 1}
_CHUNK = {"bf16": 512, "int8": 1024}  # K elements per wave-wide 16-byte load

# Tuned (waves, split) per (kind, N, K) and rows per activation-row bucket; see skinny_cfg.json.
_CFG_FILE = Path(__file__).with_name("skinny_cfg.json")
_TABLE: dict[tuple[str, int, int], dict] = {}
if _CFG_FILE.exists():
    for _key, _v in json.loads(_CFG_FILE.read_text(encoding="utf-8")).items():
        if _key.startswith("_"):
            continue
        _kind, _n, _k = _key.split("|")
        _TABLE[(_kind, int(_n), int(_k))] = _v


def _bm(m: int) -> int:
    """Activation-row bucket of a launch (M rounded up to 1, 2, 4, 8 or 16)."""
    for b in _ROW_BUCKETS:
        if m <= b:
            return b
    return ROWS_PER_LAUNCH


@functools.lru_cache(maxsize=None)
def _supported(kind: str, bm: int, rows: int, waves: int) -> bool:
    return bool(_lib.lib().bp_skinny_config_supported(_KIND_CODE[kind], bm, rows, waves))


def _default_waves(kind: str, k: int) -> int:
    nch = -(-k // _CHUNK[kind])
    waves = 1
    while waves * 2 <= min(nch, 8):
        waves *= 2
    return waves


def _default_rows(n: int, bm: int) -> int:
    rows = {1: 8, 2: 8, 4: 4, 8: 4, 16: 2}[bm]
    while rows > 2 and -(-n // rows) < 512:  # keep at least ~2 workgroups per CU on 256 CUs
        rows //= 2
    return rows


def get_cfg(kind: str, n: int, k: int, bm: int) -> tuple[int, int, int]:
    """(rows, waves, split) for a launch of `bm` activation rows; tuned table first, then the heuristic."""
    entry = _TABLE.get((kind, n, k))
    if entry is not None:
        rows = int(entry.get("rows", {}).get(str(bm), _default_rows(n, bm)))
        return rows, int(entry["waves"]), int(entry.get("split", 1))
    return _default_rows(n, bm), _default_waves(kind, k), 1


def _resolve(kind: str, n: int, k: int, bm: int, cfg) -> tuple[int, int, int]:
    """Map a user / table configuration onto the compiled menu (largest supported rows <= requested)."""
    if cfg is None:
        rows, waves, split = get_cfg(kind, n, k, bm)
    elif len(cfg) == 3:
        rows, waves, split = (int(c) for c in cfg)
    elif len(cfg) in (4, 5):  # the reference's (BN, BK, num_warps, num_stages[, split])
        rows, waves, split = int(cfg[0]), int(cfg[2]), int(cfg[4]) if len(cfg) == 5 else 1
    else:
        raise ValueError(f"cfg must be (rows, waves, split) or (BN, BK, warps, stages[, split]), got {cfg!r}")
    waves = max(w for w in _WAVES_MENU if w <= max(waves, 1))
    split = max(1, split)
    cands = [r for r in _ROWS_MENU if r <= max(rows, 2)]
    for r in sorted(cands, reverse=True):
        if _supported(kind, bm, r, waves):
            return r, waves, split
    for w in sorted((w for w in _WAVES_MENU if w < waves), reverse=True):
        for r in sorted(_ROWS_MENU, reverse=True):
            if _supported(kind, bm, r, w):
                return r, w, split
    raise ValueError(f"no compiled kernel for {kind} rows<={rows} waves<={waves} at {bm} activation rows")


MFMA_BUCKETS = (8, 16)  # row buckets (M = 5..16) served by the matrix-core kernels when the shape allows


# The LDS-staged matrix-core kernel (depth 3: each wave owns whole 16-row blocks; depth 4: the waves of a workgroup
# share each block's steps): K per 1 KiB step, activation elements a workgroup stages in LDS.
STAGED_DEPTHS = (3, 4)
STAGED_STEP = {"bf16": 512, "int8": 1024}
STAGED_K_MAX = 2048


def staged_split(kind: str, k: int, split: int = 1, waves: int = 1, depth: int = 3) -> int | None:
    """The smallest split >= `split` that the LDS-staged kernel takes for K (K / split a multiple of the step and
    at most STAGED_K_MAX; at depth 4 its steps a multiple or a divisor of the waves), or None."""
    step = STAGED_STEP[kind]
    if k <= 0 or k % step:
        return None
    for s in range(max(1, split), k // step + 1):
        if k % (s * step) == 0 and k // s <= STAGED_K_MAX:
            steps = k // s // step
            if depth != 4 or steps % waves == 0 or waves % steps == 0:
                return s
    return None


def mfma_cfg(kind: str, n: int, k: int) -> tuple[int, int, int, int] | None:
    """(block_rows, waves, depth, split) of the matrix-core kernel for a shape's 8- and 16-row buckets, or None
    when those buckets stay on the VALU kernel (table entry 'mfma', else a heuristic)."""
    if k % mfma_k_step(kind) != 0:
        return None
    entry = _TABLE.get((kind, n, k), {}).get("mfma")
    if entry is not None:
        if not entry.get("use", True):
            return None
        depth = int(entry["depth"])
        if depth in STAGED_DEPTHS and staged_split(kind, k, int(entry.get("split", 1)), int(entry["waves"]),
                                                  depth) is None:
            return None
        return int(entry["block_rows"]), int(entry["waves"]), depth, int(entry.get("split", 1))
    steps = k // mfma_k_step(kind)
    waves = 1
    while waves * 2 <= min(steps, 4):
        waves *= 2
    block_rows = 64 if n >= 32768 else 32 if n >= 4096 else 16
    return block_rows, waves, 1 if n >= 32768 else 2, 1


def _launch(kind: str, x: torch.Tensor, w: torch.Tensor, scale, y: torch.Tensor, cfg=None) -> None:
    m, k = x.shape
    n = w.shape[0]
    bm = _bm(m)
    if cfg is None and bm in MFMA_BUCKETS and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0:
        mc = mfma_cfg(kind, n, k)
        if mc is not None:
            launch_mfma(kind, x, w, scale, y, *mc)
            return
    rows, waves, split = _resolve(kind, n, k, bm, cfg)
    split = min(split, -(-k // _CHUNK[kind]))
    L = _lib.lib()
    ws = None
    ws_bytes = 0
    if split > 1:
        ws_bytes = L.bp_skinny_workspace_bytes(m, n, split)
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=x.device)
    stream = _lib.stream_ptr(x.device)
    if kind == "bf16":
        rc = L.bp_skinny_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, rows, waves, split,
                              _lib.ptr(ws), ws_bytes, stream)
    else:
        rc = L.bp_skinny_int8(x.data_ptr(), w.data_ptr(), scale.data_ptr(), _lib.TORCH_DT[scale.dtype],
                              y.data_ptr(), m, n, k, rows, waves, split, _lib.ptr(ws), ws_bytes, stream)
    _lib.check(rc, f"bp_skinny_{kind}")


def mfma_k_step(kind: str) -> int:
    """K granularity of the matrix-core kernels (K must be a multiple of it)."""
    return _mfma_k_step_cached(kind)


@functools.lru_cache(maxsize=None)
def _mfma_k_step_cached(kind: str) -> int:
    return int(_lib.lib().bp_skinny_mfma_k_step(_KIND_CODE[kind]))


def launch_mfma(kind: str, x: torch.Tensor, w: torch.Tensor, scale, y: torch.Tensor, block_rows: int, waves: int,
                depth: int = 1, split: int = 1) -> None:
    """One launch of the matrix-core kernel on 1..16 activation rows (operands validated by the caller)."""
    m, k = x.shape
    n = w.shape[0]
    if depth in STAGED_DEPTHS:
        split = staged_split(kind, k, split, waves, depth)
        if split is None:
            raise ValueError(f"K = {k} does not fit the LDS-staged matrix-core kernel")
    else:
        split = max(1, min(split, k // mfma_k_step(kind)))
    L = _lib.lib()
    ws = None
    ws_bytes = 0
    if split > 1:
        ws_bytes = L.bp_skinny_workspace_bytes(m, n, split)
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=x.device)
    stream = _lib.stream_ptr(x.device)
    if kind == "bf16":
        rc = L.bp_skinny_mfma_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, block_rows, waves, depth,
                                   split, _lib.ptr(ws), ws_bytes, stream)
    else:
        rc = L.bp_skinny_mfma_int8(x.data_ptr(), w.data_ptr(), scale.data_ptr(), _lib.TORCH_DT[scale.dtype],
                                   y.data_ptr(), m, n, k, block_rows, waves, depth, split, _lib.ptr(ws), ws_bytes,
                                   stream)
    _lib.check(rc, f"bp_skinny_mfma_{kind}")


def _check_device(x: torch.Tensor, *others: torch.Tensor | None) -> None:
    if not x.is_cuda:
        raise ValueError("x must be on a GPU (the skinny kernels have no CPU path)")
    for t in others:
        if t is not None and t.device != x.device:
            raise ValueError(f"all tensors must be on {x.device}, got {t.device}")


def skinny_mm(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor | None = None,
              zero: torch.Tensor | None = None, out: torch.Tensor | None = None,
              cfg: tuple[int, ...] | None = None) -> torch.Tensor:
    """x: [M, K] bf16 (contiguous); w: bf16 [N, K] | int8 [N, K] + scale [N]. Returns y [M, N] in x.dtype.

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
    for r0 in range(0, m, ROWS_PER_LAUNCH):
        if kind == "int4":
            _launch_int4(x[r0:r0 + ROWS_PER_LAUNCH], w, scale, zero, y[r0:r0 + ROWS_PER_LAUNCH], cfg)
        else:
            _launch(kind, x[r0:r0 + ROWS_PER_LAUNCH], w, scale, y[r0:r0 + ROWS_PER_LAUNCH], cfg)
    return y


def int4_cfg(n: int, k: int, tile_rows: int, cfg=None) -> tuple[int, int]:
    """(waves, split) of an int4 launch: the tuned table entry 'int4|N|K', else a heuristic; a user cfg is
    (waves, split) or the reference's (BN, BK, warps, stages[, split])."""
    if cfg is not None:
        if len(cfg) == 2:
            waves, split = int(cfg[0]), int(cfg[1])
        elif len(cfg) in (4, 5):
            waves, split = int(cfg[2]), int(cfg[4]) if len(cfg) == 5 else 1
        else:
            raise ValueError(f"int4 cfg must be (waves, split) or (BN, BK, warps, stages[, split]), got {cfg!r}")
    else:
        entry = _TABLE.get(("int4", n, k))
        if entry is not None:
            waves, split = int(entry["waves"]), int(entry.get("split", 1))
        else:
            groups = k // GROUP
            waves = 1
            while waves * 2 <= min(groups, 4):
                waves *= 2
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
