"""Fused on-device block selection (exact L1 score, top-k, compaction) and select+GEMM.

Reference counterpart: `_select_active_blocks` (scripts/bench_roundrobin_e2e_decode.py:90-113),
which scores blocks with the batch-mean L2 norm in fp32 and keeps `topk(...).indices.sort()`
through ~7 separate torch launches.  Here the score is the exact L1 sum
    s_j = sum_b sum_{c in block j} |x[b, 64j + c]|
(integer units of 2^-24, exact for every fp16 input), ties go to the lower block id, and the
whole selection is one kernel whose int32 output list (ascending) feeds the GEMM on the device.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from . import _lib
from ._lib import BLOCK_K, check, load
from .runtime import (_check_shapes, _dtype_code, _packed_entry, _require_cuda, _stream_handle, _views, _workspace,
                      ctypes_byref, n_keep_for_density, resolve_plan)

_SELECT_OUT_CACHE: Dict[tuple, Tuple[torch.Tensor, torch.Tensor]] = {}


def _x2d(x: torch.Tensor) -> torch.Tensor:
    x2d = x.reshape(-1, x.shape[-1])
    if x2d.stride(-1) != 1 or x2d.stride(0) % 8 != 0 or x2d.data_ptr() % 16 != 0:
        x2d = x2d.contiguous()
    return x2d


def select_topk_l1(x: torch.Tensor, k: int, idx_out: Optional[torch.Tensor] = None,
                   count_out: Optional[torch.Tensor] = None, workspace_prefix: str = "select") -> Tuple[torch.Tensor, torch.Tensor]:
    """Select min(k, nblk) blocks of x ([..., K] fp16) by exact L1 score.

    Returns (idx int32 [min(k, nblk)] ascending, count int32 [1]) — both on the device; the
    count equals min(k, nblk) and is what a device-count GEMM consumes."""
    lib = load()
    dev = _require_cuda(x)
    x2d = _x2d(x)
    bt, kd = x2d.shape
    if kd % 8 != 0:
        raise ValueError(f"K={kd} must be a multiple of 8")
    nblk = (kd + BLOCK_K - 1) // BLOCK_K
    kk = max(0, min(int(k), nblk))
    if idx_out is None:
        idx_out = torch.empty(max(kk, 1), dtype=torch.int32, device=dev)
    if count_out is None:
        count_out = torch.empty(1, dtype=torch.int32, device=dev)
    ws_bytes = int(lib.bsg_select_workspace_bytes(kd))
    ws = _workspace(workspace_prefix, dev, ws_bytes)
    with torch.cuda.device(dev):
        check(lib.bsg_select_topk_l1(x2d.data_ptr(), x2d.stride(0), bt, kd, int(k), idx_out.data_ptr(),
                                     count_out.data_ptr(), _dtype_code(x2d), ws.data_ptr(), ws_bytes,
                                     _stream_handle(dev)))
    return idx_out[:kk], count_out


def _select_active_blocks_l1(x3: torch.Tensor, density: float, block_k: int = BLOCK_K) -> torch.Tensor:
    """Drop-in for `_select_active_blocks(x3, density, block_k)` (RRD:90-113) with the exact
    L1 rule: keeps n_keep = max(1, min(nblk, round(density * nblk))) blocks, int32 ascending."""
    if int(block_k) != BLOCK_K:
        raise ValueError(f"block_k must be {BLOCK_K}")
    nblk = (x3.shape[-1] + BLOCK_K - 1) // BLOCK_K
    idx, _ = select_topk_l1(x3, n_keep_for_density(density, nblk))
    return idx


def select_sparse_gemm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, k: int, cache_prefix: str = "sel_gemm",
                       plan=None, idx_out: Optional[torch.Tensor] = None,
                       count_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused online selection + block-sparse GEMM: out = X[:, top-k blocks] · W[top-k blocks].

    x [B, S, K], weight nn.Linear [N, K], out [B, S, N].  Two launches on the current stream,
    no host round trip; returns the (device) selected list and count."""
    n_dim = out.shape[-1]
    x2d, y2d, bt, m_dim = _views(x, out, n_dim)
    _check_shapes(x2d, weight, y2d, n_dim, m_dim)
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    return select_gemm_packed(x2d, entry.packed, n_dim, k, y2d, plan=plan, idx_out=idx_out, count_out=count_out,
                              workspace_prefix=f"{cache_prefix}_ws")


def select_gemm_packed(x2d: torch.Tensor, packed: torch.Tensor, n_dim: int, k: int, y2d: torch.Tensor, plan=None,
                       idx_out: Optional[torch.Tensor] = None, count_out: Optional[torch.Tensor] = None,
                       workspace_prefix: str = "sel_gemm_ws") -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused selection + GEMM on an already packed weight: x2d [bt, K] fp16, y2d [bt, N]."""
    lib = load()
    dev = _require_cuda(x2d, packed, y2d)
    bt, m_dim = x2d.shape
    if m_dim % 8 != 0 or x2d.stride(1) != 1 or x2d.stride(0) % 8 != 0:
        raise ValueError(f"x must be [bt, K] with unit column stride and K % 8 == 0 (K={m_dim})")
    nblk = int(packed.shape[0])
    if (m_dim + BLOCK_K - 1) // BLOCK_K != nblk:
        raise ValueError(f"x has K={m_dim} but the packed weight has {nblk} K-blocks")
    kk = max(0, min(int(k), nblk))
    if idx_out is None:
        idx_out = torch.empty(max(kk, 1), dtype=torch.int32, device=dev)
    if count_out is None:
        count_out = torch.empty(1, dtype=torch.int32, device=dev)
    pl = resolve_plan(bt, n_dim, nblk, kk, dev, plan)
    sel_bytes = int(lib.bsg_select_workspace_bytes(m_dim))
    gemm_bytes = int(lib.bsg_gemm_workspace_bytes(bt, n_dim, ctypes_byref(pl)))
    ws = _workspace(workspace_prefix, dev, sel_bytes + gemm_bytes)
    with torch.cuda.device(dev):
        check(lib.bsg_select_gemm(x2d.data_ptr(), x2d.stride(0), bt, m_dim, int(k), packed.data_ptr(), n_dim,
                                  idx_out.data_ptr(), count_out.data_ptr(), y2d.data_ptr(), y2d.stride(0),
                                  _dtype_code(x2d), ws.data_ptr(), sel_bytes + gemm_bytes, ctypes_byref(pl),
                                  _stream_handle(dev)))
    return idx_out[:kk], count_out
