"""Build ``libnpu_amd.so`` (all HIP kernels + the C ABI) for gfx950 with hipcc.

Usage: ``python -m npu_amd.build`` (or ``npu_amd.build.build()``).  The library
is written next to this file, in-tree, so it travels with the source tree.
``python -m npu_amd.build --timeline`` builds the profiling variant
``libnpu_amd_tl.so`` (per-block timestamps, see csrc/timeline.h) instead.
``python -m npu_amd.build --asan`` builds ``libnpu_amd_asan.so``: the same
library with its host code (argument checks, workspace layout, error reporting)
instrumented with AddressSanitizer, for the C-ABI tests on the CPU; the device
code is built as usual.  A process loads it with the clang ASan runtime preloaded
(``asan_runtime()``) and ``NPU_AMD_LIB=asan``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libnpu_amd.so"
LIB_TL = HERE / "libnpu_amd_tl.so"
LIB_ASAN = HERE / "libnpu_amd_asan.so"
SOURCES = ["capi.hip", "matvec.hip", "router.hip", "moe_decode.hip", "moe_decode_gu.hip", "moe_decode_dn.hip",
           "dispatch.hip", "prefill.hip", "mv_bf16.hip", "core_decode.hip"]
ARCH = os.environ.get("NPU_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 ops are left to nobody: some forms have given wrong results
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


# Host-side AddressSanitizer: every sanitizer flag goes to the host compile only.
ASAN_FLAGS = ["-Xarch_host", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def is_stale(lib: Path) -> bool:
    """True when ``lib`` is missing or older than a source or header it is built from."""
    if not lib.exists():
        return True
    t = lib.stat().st_mtime
    deps = [*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *(HERE.parent / "include").glob("*.h")]
    return any(d.stat().st_mtime > t for d in deps)


def asan_runtime() -> str | None:
    """The clang ASan runtime that a process loading ``libnpu_amd_asan.so`` preloads."""
    for root in ("/opt/rocm/lib/llvm/lib/clang", "/opt/rocm/llvm/lib/clang"):
        p = Path(root)
        if p.is_dir():
            for cand in sorted(p.glob("*/lib/linux/libclang_rt.asan-x86_64.so")):
                return str(cand)
    return None


def build(verbose: bool = False, timeline: bool = False, asan: bool = False, incremental: bool = False) -> Path:
    """Compile every source to an object in parallel, then link the library
    (the timestamped profiling variant when ``timeline``, the host-only ASan
    variant when ``asan``).  ``incremental`` recompiles only the objects older
    than their source or any header."""
    objdir = HERE / ("_build_tl" if timeline else "_build_asan" if asan else "_build")
    objdir.mkdir(exist_ok=True)
    inc = ["-I", str(HERE.parent / "include")]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"] + (["-DGM_TIMELINE=1"] if timeline else [])
    if asan:
        compile_flags = compile_flags + ASAN_FLAGS
    out_lib = LIB_TL if timeline else LIB_ASAN if asan else LIB

    headers = [*CSRC.glob("*.h"), *(HERE.parent / "include").glob("*.h")]

    def fresh(obj: Path, src: Path) -> bool:
        if not (incremental and obj.exists()):
            return False
        t = obj.stat().st_mtime
        return all(d.stat().st_mtime <= t for d in (src, *headers))

    def compile_one(src: str):
        obj = objdir / (Path(src).stem + ".o")
        if fresh(obj, CSRC / src):
            return obj, subprocess.CompletedProcess([], 0, "", "")
        cmd = [hipcc(), *compile_flags, *inc, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        return obj, subprocess.run(cmd, capture_output=True, text=True)

    jobs = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(compile_one, SOURCES))
    tmp = out_lib.with_suffix(".so.tmp")
    link = [hipcc(), *HIPCC_FLAGS, *(["-Xarch_host", "-fsanitize=address"] if asan else []),
            *[str(o) for o, _ in results], "-o", str(tmp)]
    results.append((None, subprocess.run(link, capture_output=True, text=True)))
    for _, res in results:
        out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                        if "packed-fp32-ops" not in l and l.strip())
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
        if verbose and out:
            print(out)
    os.replace(tmp, out_lib)
    return out_lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, timeline="--timeline" in sys.argv, asan="--asan" in sys.argv,
                incremental="--incremental" in sys.argv))
