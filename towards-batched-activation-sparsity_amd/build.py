"""Build the gfx950 HIP library (libbsgemm.so) in-tree.

    python towards-batched-activation-sparsity_amd/build.py

The library is a plain C-ABI shared object (include/bsgemm.h) compiled with hipcc for
gfx950 only; Python reaches it through ctypes (bsa_mi355x/_lib.py).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_ROOT)
SRC = os.path.join(PKG_ROOT, "csrc", "bsgemm.hip")
INCLUDE = os.path.join(REPO_ROOT, "include")
OUT = os.path.join(PKG_ROOT, "bsa_mi355x", "libbsgemm.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    # Packed-FP32 VALU forms are kept out of every kernel (build notes).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libbsgemm.so)")


def build(verbose: bool = False) -> str:
    """Compile libbsgemm.so (always recompiles) and return its path."""
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, SRC, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
