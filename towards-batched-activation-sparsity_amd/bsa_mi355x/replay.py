"""Per-step oracle-map replay: the case construction of the reference's headline benchmark.

scripts/bench_perstep_actual_kernel_speedup.py (BPS) replays the oracle sparsity maps of
results/oracle/perstep_batch_sweep.json: for each batch size, each decode group-step holds a map
S[7 projections][32 layers] on a 0.1 grid; every (projection, layer) entry becomes one GEMM of
that projection's Llama-2-7B shape with density 1 - S and floor(density * nblk) random active
blocks (BPS:84-87, at least one).  Each distinct (shape, density) case is timed once and a
group-step's kernel-level speedup is the sum of its 224 dense times over the sum of its 224
sparse times (BPS:122-172, 210-293).  This module holds that bookkeeping; the timing lives in
bench.py (--workload perstep) and the parity check in tests/test_gpu_replay.py, so both run the
same cases.
"""
from __future__ import annotations

from typing import Dict, Iterable, List, Sequence, Tuple

import numpy as np

from ._lib import BLOCK_K

# (K, N) of each projection shape (BPS:38-51 PROJ_SHAPES / SHAPES)
SHAPES: Dict[str, Tuple[int, int]] = {"qkvo": (4096, 4096), "gate_up": (4096, 11008), "down": (11008, 4096)}
# the map's 7 rows in the reference's projection order (q, k, v, o, gate, up, down)
PROJ_SHAPE: List[str] = ["qkvo", "qkvo", "qkvo", "qkvo", "gate_up", "gate_up", "down"]


def load_maps(path: str) -> Dict[str, np.ndarray]:
    """The fixture written by tests/golden/make_perstep_fixture.py (plain arrays, no pickle)."""
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def batch_rows(fx: Dict[str, np.ndarray], bt: int) -> np.ndarray:
    """Row indices of the group-steps recorded for batch size bt."""
    return np.nonzero(fx["batch"] == bt)[0]


def density_tenths(s_tenths: int) -> int:
    """Density of a map entry, in tenths: 1 - S, clamped to [0, 1] (BPS:128)."""
    return max(0, min(10, 10 - int(s_tenths)))


def active_count(tenths: int, nblk: int) -> int:
    """max(1, min(nblk, floor(density * nblk))) for density tenths/10 (BPS:84-87), in integer
    arithmetic so no float rounding can move the floor."""
    return max(1, min(int(nblk), (int(tenths) * int(nblk)) // 10))


def nblk_of(shape: str) -> int:
    k, _ = SHAPES[shape]
    return (k + BLOCK_K - 1) // BLOCK_K


def unique_cases(maps: Iterable[np.ndarray]) -> List[Tuple[str, int]]:
    """Sorted distinct (shape, density tenths) over a set of maps ([7, 32] each)."""
    out = set()
    for m in maps:
        for pi, shape in enumerate(PROJ_SHAPE):
            for t in m[pi]:
                out.add((shape, density_tenths(t)))
    return sorted(out)


def random_blocks(rng: np.random.Generator, nblk: int, na: int) -> np.ndarray:
    """Ascending int32 ids of na distinct blocks (the seeded stand-in for BPS:87's randperm)."""
    return np.sort(rng.choice(nblk, size=int(na), replace=False)).astype(np.int32)


def step_sums(m: np.ndarray, dense_us: Dict[str, float], sparse_us: Dict[Tuple[str, int], float]) -> Tuple[float, float]:
    """(sum of dense times, sum of sparse times) over one map's 224 GEMMs."""
    d = s = 0.0
    for pi, shape in enumerate(PROJ_SHAPE):
        for t in m[pi]:
            d += dense_us[shape]
            s += sparse_us[(shape, density_tenths(t))]
    return d, s


def cases_for_batches(fx: Dict[str, np.ndarray], batches: Sequence[int], steps_per_batch: int = 0) -> Dict[int, List[Tuple[str, int]]]:
    """Distinct cases per batch size, over every group-step (steps_per_batch = 0) or the first
    steps_per_batch of them."""
    out = {}
    for bt in batches:
        rows = batch_rows(fx, bt)
        if steps_per_batch:
            rows = rows[:steps_per_batch]
        out[int(bt)] = unique_cases(fx["smap_tenths"][rows])
    return out
