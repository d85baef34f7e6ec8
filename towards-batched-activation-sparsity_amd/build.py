"""Build the gfx950 HIP library (libbsgemm.so) in-tree.

    python towards-batched-activation-sparsity_amd/build.py

The library is a plain C-ABI shared object (include/bsgemm.h) compiled with hipcc for
gfx950 only; Python reaches it through ctypes (bsa_mi355x/_lib.py).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
# The C ABI and host code, then the tile tables (each instantiates a slice of the kernel
# templates of bsg_device.hpp); the units compile in parallel and link into one library.
SOURCES = ["bsgemm.hip", "tiles_k1_r16.hip", "tiles_k1_r32.hip", "tiles_k1_r64.hip", "tiles_k2.hip",
           "tiles_k4.hip", "tiles_k3.hip", "tiles_k5.hip", "tiles_k7.hip"]
SRC = os.path.join(CSRC, "bsgemm.hip")
INCLUDE = os.path.join(REPO_ROOT, "include")
OUT = os.path.join(PKG_ROOT, "bsa_mi355x", "libbsgemm.so")
# The phase-timeline profiling build: the same sources with -DBSG_TIMELINE (per-work-group
# wall-clock stamps, include/bsgemm_timeline.h); selected at run time by BSA_MI355X_LIB=timeline.
OUT_TIMELINE = os.path.join(PKG_ROOT, "bsa_mi355x", "libbsgemm_timeline.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed-FP32 VALU forms (v_pk_*_f32) are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libbsgemm.so)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if NOISE not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd[-3:])}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 0, timeline: bool = False) -> str:
    """Compile libbsgemm.so, or with timeline=True libbsgemm_timeline.so (always recompiles every
    unit), and return its path."""
    cc = hipcc()
    jobs = jobs or min(len(SOURCES), max(1, os.cpu_count() or 1))
    out = OUT_TIMELINE if timeline else OUT
    extra = ["-DBSG_TIMELINE"] if timeline else []
    with tempfile.TemporaryDirectory(prefix="bsgemm_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[cc, *HIPCC_FLAGS, *extra, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, s), "-o", o]
                for s, o in zip(SOURCES, objs)]
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp = out + ".tmp"
        _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, timeline="--timeline" in sys.argv[1:]))
