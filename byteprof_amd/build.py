"""Build recipe of libbyteprof_amd.so: hipcc for gfx950, one object per source, objects compiled in parallel, then
linked into the shared library next to this file. `python -m byteprof_amd.build` runs it."""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB_NAME = "libbyteprof_amd.so"
LIB_PATH = PKG / LIB_NAME
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found (ROCM_PATH or PATH)")
    return found


def common_flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
            # a multiply and an add fuse only where one expression writes them (a * b + c), never across
            # statements or inlined calls: kernels that share arithmetic and must agree bit for bit round alike
            "-ffp-contract=on",
            # no packed-fp32 VALU instructions in device code
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


SOURCES = ("skinny.hip", "skinny_mf.hip", "skinny_mf_n4.hip", "skinny_mf_n8.hip", "skinny_mf_n16.hip",
           "skinny_chain.hip", "skinny_int4.hip", "mlstm.hip", "draft.hip", "decode.hip")


def units() -> list[tuple[Path, list[str], Path]]:
    """(source, extra flags, object) for every translation unit."""
    return [(CSRC / name, [], BUILD_DIR / name.replace(".hip", ".o")) for name in SOURCES]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only target feature; that warning is expected
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every HIP source and link the library; always rebuilds. Returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    cmds = [[cc, *common_flags(), *extra, "-c", str(src), "-o", str(obj)] for src, extra, obj in units()]
    jobs = jobs or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for _, _, o in units()]]
    _run(link)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


TIMELINE_LIB_PATH = PKG / "libbyteprof_amd_timeline.so"
# the units with timeline stamps (compiled with -DBP_TIMELINE)
TIMELINE_SOURCES = ("mlstm.hip", "skinny_mf.hip", "skinny_mf_n4.hip", "skinny_mf_n8.hip", "skinny_mf_n16.hip")


def build_timeline(verbose: bool = False) -> Path:
    """The timeline library: the units of TIMELINE_SOURCES compiled with -DBP_TIMELINE, linked with the normal
    objects of the others (build() first). Same C ABI plus the timeline readers; for profiling only."""
    cc = hipcc()
    objs, cmds = [], []
    for src, extra, obj in units():
        if src.name in TIMELINE_SOURCES:
            tl_obj = obj.with_name(obj.stem + "_timeline.o")
            cmds.append([cc, *common_flags(), *extra, "-DBP_TIMELINE", "-c", str(src), "-o", str(tl_obj)])
            objs.append(tl_obj)
        else:
            if not obj.exists():
                raise RuntimeError(f"{obj} is missing: run build() first")
            objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
    tmp = TIMELINE_LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for o in objs]])
    os.replace(tmp, TIMELINE_LIB_PATH)
    return TIMELINE_LIB_PATH


if __name__ == "__main__":
    if "--timeline" in sys.argv:
        print(build_timeline(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
