"""Properties of the generated gfx950 code that the kernels' correctness or speed rests on and
that no result test can pin reliably (CPU only: hipcc cross-compiles the device code to assembly).

- Kind 7 waits for its LDS-bound activation loads by count, which is right only if each pipeline
  slot issues all of its activation loads before its weight loads and before the next slot's:
  the compiler's scheduler is free to interleave them unless told not to, and a wrong order is a
  race that a fast L2 usually hides.
- Kinds 5/6 keep their main loops free of full pipeline drains (`s_waitcnt vmcnt(0)` inside a
  loop that runs MFMAs) except in the four tiles where the register allocator is known to force
  one; unrelated edits to the shared device code have added drains to other tiles before.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "towards-batched-activation-sparsity_amd", "csrc")


def _hipcc():
    for c in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"), shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


def _device_asm(unit: str, tmp_path) -> str:
    cc = _hipcc()
    if cc is None:
        pytest.skip("hipcc not available")
    out = os.path.join(str(tmp_path), unit + ".s")
    cmd = [cc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           "--cuda-device-only", "-S", "-o", out, os.path.join(CSRC, unit)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return open(out).read()


def _functions(asm: str, prefix: str):
    for name in re.findall(r"^(" + prefix + r"\w*):", asm, re.M):
        i = asm.index(name + ":")
        yield name, asm[i:asm.index(".Lfunc_end", i)].split("\n")


def test_lds_activation_kernels_issue_each_slot_in_order(tmp_path):
    asm = _device_asm("tiles_k7.hip", tmp_path)
    checked = 0
    for name, body in _functions(asm, "_ZN12_GLOBAL__N_119bsg_gemm_vtx_kernel"):
        btt, nsub = [int(a) for a in re.findall(r"Li(\d+)E", name)][:2]
        seq = "".join("X" if " lds" in line else "W" for line in body
                      if "buffer_load_dwordx4" in line and (" lds" in line or " nt" in line))
        runs = re.findall(r"X+|W+", seq)
        assert runs, name
        for k, r in enumerate(runs):
            assert r[0] == ("X" if k % 2 == 0 else "W") and len(r) == (2 * btt if r[0] == "X" else 2 * nsub), \
                (name, [len(x) for x in runs])
        checked += 1
    assert checked >= 30


def _drains_in_mfma_loops(body) -> bool:
    labels = {}
    for k, line in enumerate(body):
        m = re.match(r"^(\.LBB\d+_\d+):", line.strip())
        if m:
            labels[m.group(1)] = k
    for k, line in enumerate(body):
        m = re.match(r"\s*s_cbranch_\w+\s+(\.LBB\d+_\d+)", line) or re.match(r"\s*s_branch\s+(\.LBB\d+_\d+)", line)
        if m and m.group(1) in labels and labels[m.group(1)] < k:
            loop = body[labels[m.group(1)]:k + 1]
            if sum("v_mfma" in x for x in loop) >= 4 and any("vmcnt(0)" in x for x in loop):
                return True
    return False


def test_variable_width_kernels_keep_their_loops_free_of_drains(tmp_path):
    asm = _device_asm("tiles_k5.hip", tmp_path)
    # kind 6 tiles (rows / 16, subtiles, waves, depth) whose loops are known to drain once per slot
    known = {(1, 1, 4, 8), (1, 2, 4, 8), (2, 1, 8, 4), (2, 2, 8, 4)}
    names = 0
    for name, body in _functions(asm, "_ZN12_GLOBAL__N_118bsg_gemm_vt_kernel"):
        names += 1
        if _drains_in_mfma_loops(body):
            btt, nsub, wb, depth, kh = [int(a) for a in re.findall(r"Li(\d+)E", name)][:5]
            assert kh == 1 and (btt, nsub, wb, depth) in known, name
    assert names >= 100
