"""Mutation check of the GPU tests: plausible bugs planted in copies of the kernel sources (and one in the host-side
int4 packing), each built into its own library, then the skinny GPU tests run against every mutant; a mutant is
killed when at least one test fails.

The mutants restate the reference's kernel mutants (byteprof tools/skinny_mutation.py:12-26) for this build's HIP
sources, plus three of the matrix-core layout. Every mutant keeps all memory accesses in bounds, so none can fault
the GPU:
  - where the reference's mutant would read or write past a buffer, the same bug is planted in an in-bounds form
    ("split-K ranges overlap" as ranges shifted by one segment; "K tail not masked" as a tail mask that drops the
    last element; "output rows transposed" as the row order reversed);
  - "store not masked on rows >= M" writes past y whatever form it takes; it is listed and not run.

Usage:
  python tests/mutation.py build   # where hipcc is: compiles the mutated translation units, links one library per
                                   # mutant under byteprof_amd/_mutants/ (needs a current `python -m byteprof_amd.build`)
  python tests/mutation.py run [name ...]
                                   # on the GPU: the unmutated sources, then each mutant (or those whose name
                                   # contains a given word; their results replace the earlier ones); writes
                                   # tests/mutation_results.json. Kernel mutants are judged by the GPU tests of the
                                   # skinny path, the host-side mutant also by the CPU tests of the same code.
"""

from __future__ import annotations

import json
import os
import re
import shutil
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "byteprof_amd"
OUT = PKG / "_mutants"
OBJ = PKG / "_build" / "mutants"
RESULTS = Path(__file__).resolve().parent / "mutation_results.json"
TESTS = ["tests/test_skinny_gpu.py", "tests/test_int8_gpu.py", "tests/test_int4_gpu.py", "tests/test_configs_gpu.py",
         "tests/test_prologue_gpu.py"]

# (name, file under byteprof_amd/, old text, new text); new None: listed, not run (the reason in old)
MUTANTS = [
    ("int4 nibble halves swapped", "csrc/skinny_int4.hip",
     "const int sh = c < 2 ? 0 : 4;", "const int sh = c < 2 ? 4 : 0;"),
    ("int4 zero offset 127 instead of 128", "csrc/skinny_int4.hip",
     "acc[h][r] += sc * (D[r] - (128.f + z) * X[r]);", "acc[h][r] += sc * (D[r] - (127.f + z) * X[r]);"),
    ("int4 group scale ignored", "csrc/skinny_int4.hip",
     "acc[h][r] += sc * (D[r] - (128.f + z) * X[r]);", "acc[h][r] += (D[r] - (128.f + z) * X[r]);"),
    ("int8 channel scale ignored", "csrc/skinny_mf_kernel.h",
     "if constexpr (KIND == kInt8) t *= row_scale(0);\n        yk[",
     "if constexpr (KIND == kInt8) t *= 1.f;\n        yk["),
    ("split-K reduce skips the last split", "csrc/skinny.hip",
     "for (int s = 1; s < split; ++s) t += ws[s * total + idx];",
     "for (int s = 1; s < split - 1; ++s) t += ws[s * total + idx];"),
    ("split-K ranges overlap (shifted by one segment)", "csrc/skinny_mf_kernel.h",
     "const int64_t s_lo = split == 1 ? 0 : sp * nseg_all / split;\n"
     "  const int64_t s_hi = split == 1 ? nseg_all : (sp + 1) * nseg_all / split;",
     "const int64_t s_lo = split == 1 ? 0 : sp * nseg_all / split - (sp > 0);\n"
     "  const int64_t s_hi = split == 1 ? nseg_all : (sp + 1) * nseg_all / split - (sp > 0);"),
    ("K tail mask drops the last element (bf16 element loads)", "csrc/skinny_mf.h",
     "if (k + e < K) d[e >> 1] |= static_cast<uint32_t>(p[k + e]) << (16 * (e & 1));",
     "if (k + e < K - 1) d[e >> 1] |= static_cast<uint32_t>(p[k + e]) << (16 * (e & 1));"),
    ("row bucket too small (17 rows in a 16-row block)", "csrc/skinny_mf.hip",
     "int mf_blocks(int64_t M) { return M <= 8 ? 1 : M <= 16 ? 2 : M <= 32 ? 4 : 8; }",
     "int mf_blocks(int64_t M) { return M <= 8 ? 1 : M <= 17 ? 2 : M <= 32 ? 4 : 8; }"),
    ("store not masked on rows >= M", "csrc/skinny_mf_kernel.h",
     "not run: every form of it writes rows past y's [M, N]", None),
    ("output rows reversed", "csrc/skinny_mf_kernel.h",
     "yk[static_cast<int64_t>(m) * N + n] = float_to_bf16_bits(t);",
     "yk[static_cast<int64_t>(m) * N + (N - 1 - n)] = float_to_bf16_bits(t);"),
    ("activation operands one piece late (buffer offsets)", "csrc/skinny_mf.h",
     "const uint32_t o = off[b] + static_cast<uint32_t>(2 * (s * G::kSeg + 8 * part));",
     "const uint32_t o = off[b] + static_cast<uint32_t>(2 * (s * G::kSeg + 8 * part + 8));"),
    ("int4 pack: high nibble from the low code", "optim/skinny.py",
     "g[:, :, :, 0] | (g[:, :, :, 1] << 4)", "g[:, :, :, 0] | (g[:, :, :, 0] << 4)"),
    ("MFMA halves folded from the wrong lanes", "csrc/skinny_mf.h",
     "v.x += __shfl_down(v.x, 40);", "v.x += __shfl_down(v.x, 32);"),
    ("int8 weights read as unsigned bytes", "csrc/common.h",
     "const float lo = static_cast<float>(static_cast<int8_t>(d >> sh));",
     "const float lo = static_cast<float>(static_cast<uint8_t>(d >> sh));"),
    ("bf16 outputs truncated instead of rounded to nearest even", "csrc/common.h",
     "return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));",
     "return static_cast<uint16_t>(__float_as_uint(f) >> 16);"),
]


def _slug(name: str) -> str:
    return re.sub(r"[^a-z0-9]+", "_", name.lower()).strip("_")[:48]


def _includes(path: Path) -> set[str]:
    return set(re.findall(r'#include "([^"]+)"', path.read_text()))


def _units_touching(mutated: str) -> list[str]:
    """The library's translation units whose include graph reaches the mutated csrc file."""
    from byteprof_amd import build as B

    csrc = PKG / "csrc"
    out = []
    for src in B.SOURCES:
        seen, todo = set(), [src]
        while todo:
            f = todo.pop()
            if f in seen or not (csrc / f).exists():
                continue
            seen.add(f)
            todo.extend(_includes(csrc / f))
        if mutated in seen:
            out.append(src)
    return out


def build() -> int:
    sys.path.insert(0, str(ROOT))
    from byteprof_amd import build as B

    base_objs = {src: B.BUILD_DIR / src.replace(".hip", ".o") for src in B.SOURCES}
    missing = [str(o) for o in base_objs.values() if not o.exists()]
    if missing:
        print(f"build the library first (python -m byteprof_amd.build): missing {missing}", file=sys.stderr)
        return 1
    OUT.mkdir(exist_ok=True)
    cc = B.hipcc()
    for name, rel, old, new in MUTANTS:
        if new is None or not rel.startswith("csrc/"):
            continue
        slug = _slug(name)
        work = OBJ / slug
        shutil.rmtree(work, ignore_errors=True)
        shutil.copytree(PKG / "csrc", work / "csrc")
        target = work / rel
        text = target.read_text()
        if text.count(old) != 1:
            print(f"{name}: the mutated text occurs {text.count(old)} times in {rel}", file=sys.stderr)
            return 1
        target.write_text(text.replace(old, new))
        units = _units_touching(Path(rel).name)
        objs = dict(base_objs)
        flags = [f for f in B.common_flags() if not f.startswith("-I")]
        for src in units:
            obj = work / src.replace(".hip", ".o")
            B._run([cc, *flags, f"-I{B.INCLUDE}", f"-I{work / 'csrc'}", "-c", str(work / "csrc" / src), "-o", str(obj)])
            objs[src] = obj
        lib = OUT / f"lib_{slug}.so"
        B._run([cc, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-o", str(lib), *[str(o) for o in objs.values()]])
        print(f"{name}: rebuilt {', '.join(units)} -> {lib.relative_to(ROOT)}", flush=True)
    return 0


# Host-side mutants are also judged by the CPU tests of the same code (run without the gpu marker: on a machine
# without a GPU the GPU tests skip themselves).
HOST_TESTS = ["tests/test_host.py", "tests/test_oracle.py"]


def _files(rel: str) -> tuple[list[str], bool]:
    """The test files a mutant of `rel` is judged by, and whether to select only GPU tests."""
    return (TESTS, True) if rel.startswith("csrc/") else (HOST_TESTS + TESTS, False)


def _pytest(env: dict, files: list[str], gpu_only: bool) -> tuple[int, str, float]:
    t0 = time.perf_counter()
    marker = ["-m", "gpu"] if gpu_only else []
    r = subprocess.run([sys.executable, "-u", "-m", "pytest", "-x", "-q", *marker, "--timeout", "120",
                        "--timeout-method", "thread", *files], cwd=ROOT, env=env, capture_output=True, text=True)
    lines = [ln for ln in r.stdout.strip().splitlines() if ln.strip()]
    return r.returncode, (lines[-1] if lines else r.stderr[-300:]), time.perf_counter() - t0


def run(only: list[str]) -> int:
    """Every mutant (or those whose name contains one of `only`; their results replace the earlier ones in the
    results file)."""
    env = {k: v for k, v in os.environ.items() if k != "BYTEPROF_AMD_LIB"}
    chosen = [m for m in MUTANTS if not only or any(o in m[0] for o in only)]
    baselines = {}
    for _, rel, _, new in chosen:
        files, gpu_only = _files(rel)
        key = (tuple(files), gpu_only)
        if new is None or key in baselines:
            continue
        print(f"[mutation] unmutated sources, {' '.join(files)}", flush=True)
        rc, last, sec = _pytest(env, files, gpu_only)
        print(f"[mutation] unmutated: rc {rc} ({last}) in {sec:.0f} s", flush=True)
        if rc != 0:
            print("the unmutated sources fail the tests: no mutant can be judged", file=sys.stderr)
            return 1
        baselines[key] = last
    res = []
    for name, rel, old, new in chosen:
        if new is None:
            res.append({"mutant": name, "file": rel, "killed": None, "note": old})
            print(f"[mutation] {name}: {old}", flush=True)
            continue
        print(f"[mutation] {name}", flush=True)
        files, gpu_only = _files(rel)
        if rel.startswith("csrc/"):
            lib = OUT / f"lib_{_slug(name)}.so"
            if not lib.exists():
                res.append({"mutant": name, "file": rel, "killed": None, "note": "library not built"})
                continue
            rc, last, sec = _pytest({**env, "BYTEPROF_AMD_LIB": str(lib)}, files, gpu_only)
        else:  # host-side Python: planted in place, restored afterwards
            path = PKG / rel
            orig = path.read_text()
            if orig.count(old) != 1:
                res.append({"mutant": name, "file": rel, "killed": None, "note": "pattern not found"})
                continue
            stale = lambda: [c.unlink() for c in (path.parent / "__pycache__").glob(path.stem + ".*.pyc")]  # noqa: E731
            try:
                path.write_text(orig.replace(old, new))
                stale()  # the same size and second as the original: a cached compilation would hide the change
                rc, last, sec = _pytest(env, files, gpu_only)
            finally:
                path.write_text(orig)
                stale()
        # rc 1: tests failed (killed); 0: survived; anything else (a crash, an interrupted run) is recorded as is
        killed = True if rc == 1 else False if rc == 0 else None
        res.append({"mutant": name, "file": rel, "killed": killed, "pytest_rc": rc, "last_line": last,
                    "tests": files, "gpu_only": gpu_only, "seconds": round(sec, 1)})
        print(f"[mutation] {name}: {'killed' if killed else 'SURVIVED' if killed is False else f'rc {rc}'} ({last})",
              flush=True)
    if only and RESULTS.exists():
        merged = {m["mutant"]: m for m in json.loads(RESULTS.read_text())["mutants"]}
        merged.update({m["mutant"]: m for m in res})
        res = [merged[name] for name, *_ in MUTANTS if name in merged]
    RESULTS.write_text(json.dumps({"mutants": res}, indent=1) + "\n")
    n_run = sum(r["killed"] is not None for r in res)
    print(f"[mutation] killed {sum(r['killed'] is True for r in res)} of {n_run} run", flush=True)
    return 0


if __name__ == "__main__":
    if len(sys.argv) < 2 or sys.argv[1] not in ("build", "run") or (sys.argv[1] == "build" and len(sys.argv) > 2):
        print(__doc__, file=sys.stderr)
        sys.exit(2)
    sys.exit(build() if sys.argv[1] == "build" else run(sys.argv[2:]))
