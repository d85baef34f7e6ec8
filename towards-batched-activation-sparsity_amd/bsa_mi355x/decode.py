"""A Llama-2-7B-shaped decode step of linears, captured as one hipGraph.

Per layer, in the model's order (q/k/v share their input and mask, as do gate/up, so each pair
or triple runs as one GEMM over the concatenated output columns, like the fused-QKV shape of
kernels/shared_mask_batched_triton_min_runtime.py:4301):

    select(x_attn) -> qkv  GEMM  (K=4096,  N=3*4096)
    select(x_o)    -> o    GEMM  (K=4096,  N=4096)
    select(x_mlp)  -> gate/up GEMM (K=4096, N=2*11008)
    select(x_down) -> down GEMM  (K=11008, N=4096)

Every select is the exact-L1 top-k on that projection's input (a block-score launch, then the
GEMM ranks the scores itself, or a rank launch precedes it); the list stays on the device (no
host round trip), so the whole step -- 32 layers x 4 x (select + GEMM) -- is one graph.  Attention, norms and activations are outside this path: the four inputs
of each layer are fixed synthetic activations, and weights are random with
the Llama-2-7B architecture's shapes (~13 GB packed, resident in HBM).
"""
from __future__ import annotations

from typing import List, Optional

import torch

from ._lib import BLOCK_K
from .runtime import n_keep_for_density, pack_weight
from .select import select_gemm_packed

HIDDEN = 4096
INTERMEDIATE = 11008
N_LAYERS = 32

# name, K, N (fused output columns)
PROJECTIONS = [("qkv", HIDDEN, 3 * HIDDEN), ("o", HIDDEN, HIDDEN), ("gate_up", HIDDEN, 2 * INTERMEDIATE),
               ("down", INTERMEDIATE, HIDDEN)]


class _Proj:
    def __init__(self, name: str, k: int, n: int, packed: torch.Tensor, x: torch.Tensor, keep: int):
        self.name, self.k, self.n = name, k, n
        self.packed = packed
        self.x = x
        self.keep = keep
        self.nblk = (k + BLOCK_K - 1) // BLOCK_K
        self.y = torch.empty(x.shape[0], n, dtype=x.dtype, device=x.device)
        self.idx = torch.empty(max(keep, 1), dtype=torch.int32, device=x.device)
        self.cnt = torch.empty(1, dtype=torch.int32, device=x.device)

    @property
    def active_bytes(self) -> int:
        return min(self.keep, self.nblk) * BLOCK_K * self.n * 2


class DecodeStep:
    """Holds packed weights, inputs and outputs of an n_layers-deep decode step of linears."""

    def __init__(self, batch: int = 64, density: float = 0.48, n_layers: int = N_LAYERS,
                 device: Optional[torch.device] = None, seed: int = 1234, dtype=torch.float16):
        self.device = device or torch.device("cuda", torch.cuda.current_device())
        self.batch, self.density, self.n_layers = batch, density, n_layers
        g = torch.Generator(device=self.device).manual_seed(seed)
        self.layers: List[List[_Proj]] = []
        for _ in range(n_layers):
            projs = []
            for name, k, n in PROJECTIONS:
                # W ~ N(0, 0.02) generated as [K, N] on the device, packed, then dropped
                w = (torch.randn(k, n, generator=g, device=self.device, dtype=torch.float32) * 0.02).to(dtype)
                packed = pack_weight(w, layout="kn")
                del w
                if name == "down":
                    u = torch.rand(batch, k, generator=g, device=self.device) - 0.5
                    x = (-0.05 * torch.sign(u) * torch.log1p(-2 * u.abs())).to(dtype)  # Laplace(0, 0.05)
                else:
                    x = torch.randn(batch, k, generator=g, device=self.device).to(dtype)
                keep = n_keep_for_density(density, (k + BLOCK_K - 1) // BLOCK_K)
                projs.append(_Proj(name, k, n, packed, x, keep))
            self.layers.append(projs)
        torch.cuda.synchronize(self.device)
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    @property
    def resident_weight_bytes(self) -> int:
        return sum(p.packed.numel() * p.packed.element_size() for layer in self.layers for p in layer)

    @property
    def active_bytes(self) -> int:
        return sum(p.active_bytes for layer in self.layers for p in layer)

    def projections(self):
        for li, layer in enumerate(self.layers):
            for p in layer:
                yield li, p

    def run(self) -> None:
        """Enqueue the whole step on the current stream (eager)."""
        for li, p in self.projections():
            select_gemm_packed(p.x, p.packed, p.n, p.keep, p.y, idx_out=p.idx, count_out=p.cnt,
                               workspace_prefix=f"decode_{li}_{p.name}")

    def capture(self) -> torch.cuda.CUDAGraph:
        """Warm up (workspaces, plans) then capture the step as one graph."""
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self.run()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run()
        torch.cuda.synchronize(self.device)
        self.graph = g
        return g

    def replay(self) -> None:
        if self.graph is None:
            self.capture()
        self.graph.replay()
