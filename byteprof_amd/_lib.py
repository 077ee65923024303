"""ctypes binding of libbyteprof_amd.so (the C ABI declared in include/byteprof_amd.h).

torch is imported before the library is loaded, so the library's `libamdhip64.so.7` dependency resolves to the HIP
runtime torch already mapped: the streams and device pointers torch hands out are then valid in the library. The
loader checks that exactly one HIP runtime is mapped. There is no fallback: if the library is missing or fails to
load, every call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the library load: shares torch's HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "libbyteprof_amd.so"
# BYTEPROF_AMD_LIB: another build of the same ABI to load instead (the mutation check, tests/mutation.py)
LIB_ENV = "BYTEPROF_AMD_LIB"

BP_OK = 0
BP_E_INVALID_ARG = -1
BP_E_UNSUPPORTED = -2
BP_E_WORKSPACE = -3

DT_BF16, DT_F16, DT_F32, DT_I8 = 0, 1, 2, 3
TORCH_DT = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32, torch.int8: DT_I8}

_c_i64, _c_int, _c_size, _c_vp, _c_float = ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes); mirrors include/byteprof_amd.h
SIGNATURES: dict[str, tuple] = {
    "bp_version": (_c_int, []),
    "bp_status_string": (ctypes.c_char_p, [_c_int]),
    "bp_skinny_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_int]),
    "bp_skinny_mf_supported": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "bp_skinny_mf_k_segment": (_c_int, [_c_int]),
    "bp_skinny_mf_stage_bytes": (_c_i64, [_c_int, _c_i64, _c_i64, _c_int]),
    "bp_skinny_mf_stage_bytes_rows": (_c_i64, [_c_int, _c_i64, _c_i64, _c_int, _c_int]),
    "bp_skinny_mf": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int,
                              _c_int, _c_vp, _c_size, _c_vp]),
    "bp_skinny_mf_partials": (_c_int, [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                       _c_vp, _c_size, _c_vp]),
    "bp_skinny_mf_silu": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                   _c_int, _c_vp]),
    "bp_skinny_mf_static_bytes": (_c_size, []),
    "bp_skinny_mf_static": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                     _c_int, _c_int, _c_vp]),
    "bp_skinny_mf_pro": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                  _c_int, _c_vp, _c_vp]),
    "bp_chain_supported": (_c_int, [_c_int, _c_int, _c_int]),
    "bp_chain_scratch_bytes": (_c_size, [_c_int]),
    "bp_chain_plan": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_int]),
    "bp_chain_run": (_c_int, [_c_int, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp, _c_int, _c_vp]),
    "bp_skinny_int4_config_supported": (_c_int, [_c_int, _c_int, _c_int]),
    "bp_skinny_int4": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                _c_int, _c_vp, _c_size, _c_vp]),
    "bp_skinny_int4_silu": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                                     _c_int, _c_vp]),
    "bp_skinny_int4_pro": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                                    _c_int, _c_int, _c_vp, _c_vp]),
    "bp_splitk_reduce": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_int, _c_vp]),
    "bp_mlstm_multistep": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                    _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                    _c_float, _c_float, _c_int, _c_vp]),
    "bp_mlstm_step": (_c_int, [_c_vp] * 12 + [_c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_int,
                                                _c_vp]),
    "bp_mlstm_lazy_commit": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                      _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                      _c_int, _c_vp]),
    "bp_draft_accept": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp]),
    "bp_draft_commit": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_vp]),
    "bp_decode_embed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_i64, _c_vp]),
    "bp_decode_qk_rope_cache": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int,
                                         _c_int, _c_float, _c_vp]),
    "bp_decode_attention": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_float, _c_vp]),
    "bp_decode_rope_attention": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int,
                                          _c_int, _c_float, _c_float, _c_vp]),
    "bp_decode_rope_attention_rows": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int,
                                               _c_int, _c_int, _c_int, _c_float, _c_float, _c_vp]),
    "bp_decode_splitk_norm_residual_rows": (_c_int, [_c_vp, _c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_int,
                                                     _c_float, _c_int, _c_vp]),
    "bp_decode_norm_residual": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_float, _c_vp]),
    "bp_decode_silu_mul": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp]),
    "bp_decode_argmax_scratch_bytes": (_c_size, []),
    "bp_decode_argmax_next": (_c_int, [_c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_vp]),
    "bp_decode_embed_rows": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_i64, _c_vp]),
    "bp_decode_qk_rope_cache_rows": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int,
                                              _c_int, _c_float, _c_int, _c_vp]),
    "bp_decode_attention_rows": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_float, _c_int,
                                          _c_vp]),
    "bp_decode_norm_residual_rows": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_float, _c_int, _c_vp]),
    "bp_decode_silu_mul_rows": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp]),
    "bp_decode_argmax_rows_scratch_bytes": (_c_size, [_c_int]),
    "bp_decode_argmax_rows": (_c_int, [_c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "bp_draft_verify_next": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp]),
}

_LIB: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """A bp_* call returned a non-zero status."""


def _mapped_hip_runtimes() -> set[str]:
    try:
        with open("/proc/self/maps", encoding="utf-8") as fh:
            return {os.path.realpath(line.split()[-1]) for line in fh if "libamdhip64" in line}
    except OSError:
        return set()


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use). Raises RuntimeError if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ[LIB_ENV]) if os.environ.get(LIB_ENV) else LIB_PATH
    if not path.exists():
        raise RuntimeError(f"{path} is not built: run `python -m byteprof_amd.build` "
                           "(or __graft_entry__.build()) first")
    handle = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    runtimes = _mapped_hip_runtimes()
    if len(runtimes) > 1:
        raise RuntimeError(f"more than one HIP runtime is mapped ({sorted(runtimes)}); "
                           "import torch before loading libbyteprof_amd.so")
    _LIB = handle
    return handle


def check(status: int, what: str) -> None:
    if status != BP_OK:
        msg = lib().bp_status_string(status).decode()
        raise NativeError(f"{what} failed with status {status}: {msg}")


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`, as an integer."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
