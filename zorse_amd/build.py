"""Build recipe for libzorse_amd.so (gfx950).

Each ``csrc/*.hip`` file is compiled to an object with hipcc (in parallel),
then linked into ``zorse_amd/libzorse_amd.so``.  The library depends only on
the HIP runtime; when it is loaded after ``import torch`` the dynamic loader
binds it to the HIP runtime torch already mapped (same SONAME), so torch's
streams and allocations are shared with the kernels.

Usage: ``python -m zorse_amd.build`` or ``zorse_amd.build.build()``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libzorse_amd.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops stay disabled for every kernel in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source extra flags.  rope.hip: with packed fp32 disabled, the SLP
# vectoriser forms two-wide fp32 negations that this compiler cannot select
# (a backend "Cannot select: v2f32 bitcast" crash in the position-major
# kernel); the kernels there are memory-bound, so scalar code costs nothing.
# gemm.hip, gemm_kmajor.hip: the GEMM's LDS-DMA asm declares M0 clobbered,
# which clang reports as a clobber of a reserved register (the intent: the
# compiler keeps nothing in M0 across the asm).  gemm_kmajor.hip (the tiled
# forms with a K-major operand): the greedy register allocator assigns local
# live ranges in reverse order, which keeps the 256 accumulators in place
# through the loop (with the default order the both-K-major form moved ~80
# of them between AGPRs per pass; the NT forms do better with the default).
FILE_FLAGS = {"rope.hip": ["-fno-slp-vectorize"], "gemm.hip": ["-Wno-inline-asm"],
              "gemm_kmajor.hip": ["-Wno-inline-asm", "-mllvm", "-greedy-reverse-local-assignment=1"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every kernel source and link the shared library.  Always
    rebuilds (the driver's build check compiles from source each time)."""
    hipcc = _hipcc()
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))

    def compile_one(pair):
        src, obj = pair
        cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src,
               "-o", obj]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    _run(cmd)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
