"""Per-step oracle-map replay: the case construction of the reference's headline benchmark.

scripts/bench_perstep_actual_kernel_speedup.py (BPS) replays the oracle sparsity maps of
results/oracle/perstep_batch_sweep.json: for each batch size, each decode group-step holds a map
S[7 projections][32 layers] on a 0.1 grid; every (projection, layer) entry becomes one GEMM of
that projection's Llama-2-7B shape with density 1 - S and floor(density * nblk) random active
blocks (BPS:84-87, at least one).  Each distinct (shape, density) case is timed once and a
group-step's kernel-level speedup is the sum of its 224 dense times over the sum of its 224
sparse times (BPS:122-172, 210-293).  This module holds that bookkeeping; the timing lives in
bench.py (--workload perstep) and the parity check in tests/test_gpu_replay.py, so both run the
same cases.  StepGraphs also runs a group-step's 224 GEMMs as one captured graph, so the step is
timed whole (launch intervals and cache state included) instead of as a sum of per-case times.
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


class StepGraphs:
    """The 224-GEMM decode step of one group-step's map as one hipGraph (the oracle-map replay
    as a whole step rather than per case): 32 layers x the 7 projections in the reference's order (q, k, v,
    o, gate, up, down; BPS:122-141), each layer with its own random-init weights (the Llama-2-7B
    step's ~13 GB, more than the 256 MB Infinity Cache can hold, so no rotation is needed), each
    GEMM with floor(density * nblk) random active blocks from the map entry (BPS:84-87).  The
    dense step is the same 224 launches with every block active.  Inputs are one synthetic X per
    projection shape and batch size (the reference's per-case x, BPS:148-160); every GEMM writes
    its own Y.  The weights are built once; set_batch() switches X and Y to another batch size."""

    N_LAYERS = 32

    def __init__(self, device, n_layers: int = N_LAYERS, seed: int = 1234, dtype=None):
        import torch

        from .runtime import pack_weight

        self.device, self.n_layers, self.seed = device, int(n_layers), int(seed)
        self.dtype = dtype or torch.float16
        g = torch.Generator(device=device).manual_seed(seed)
        # packed[layer][projection index]
        self.packed = []
        for _ in range(self.n_layers):
            row = []
            for shape in PROJ_SHAPE:
                k, n = SHAPES[shape]
                w = (torch.randn(k, n, generator=g, device=device, dtype=torch.float32) * 0.02).to(self.dtype)
                row.append(pack_weight(w, layout="kn"))
                del w
            self.packed.append(row)
        torch.cuda.synchronize(device)
        self.batch = 0

    @property
    def resident_weight_bytes(self) -> int:
        return sum(p.numel() * p.element_size() for row in self.packed for p in row)

    def set_batch(self, batch: int) -> None:
        import torch

        self.batch = int(batch)
        g = torch.Generator(device=self.device).manual_seed(self.seed + self.batch)
        self.x = {s: torch.randn(self.batch, k, generator=g, device=self.device).to(self.dtype)
                  for s, (k, _) in SHAPES.items()}
        self.y = [[torch.empty(self.batch, SHAPES[s][1], dtype=self.dtype, device=self.device) for s in PROJ_SHAPE]
                  for _ in range(self.n_layers)]

    def step_lists(self, m: np.ndarray, rng: np.random.Generator):
        """Per (layer, projection) ascending int32 device lists for one map [7, 32] (sparsity
        tenths), drawn from rng in layer-major order."""
        import torch

        out = []
        for li in range(self.n_layers):
            row = []
            for pi, shape in enumerate(PROJ_SHAPE):
                nb = nblk_of(shape)
                na = active_count(density_tenths(m[pi][li]), nb)
                row.append(torch.from_numpy(random_blocks(rng, nb, na)).to(self.device))
            out.append(row)
        return out

    def active_bytes(self, lists=None) -> int:
        """Active-weight bytes of one step (lists None: the dense step)."""
        total = 0
        for li in range(self.n_layers):
            for pi, shape in enumerate(PROJ_SHAPE):
                na = nblk_of(shape) if lists is None else int(lists[li][pi].numel())
                total += na * BLOCK_K * SHAPES[shape][1] * 2
        return total

    def run(self, lists=None) -> None:
        """Enqueue the step on the current stream: lists[layer][proj] (None: the dense step)."""
        from .runtime import gemm_packed, resolve_plan

        for li in range(self.n_layers):
            for pi, shape in enumerate(PROJ_SHAPE):
                _, n = SHAPES[shape]
                nb = nblk_of(shape)
                idx = None if lists is None else lists[li][pi]
                na = nb if idx is None else int(idx.numel())
                plan = resolve_plan(self.batch, n, nb, na, self.device, None, dense=idx is None)
                gemm_packed(self.x[shape], self.packed[li][pi], n, idx, self.y[li][pi], plan=plan,
                            workspace_prefix=f"stepgraph_{shape}_{pi}")

    def capture(self, lists=None):
        """Warm up (plans, workspaces) on a side stream, then capture the step as one graph."""
        import torch

        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self.run(lists)
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.run(lists)
        torch.cuda.synchronize(self.device)
        return graph
