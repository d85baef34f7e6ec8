"""2-D block sparsity: active K-blocks *and* active 64-column output blocks.

Reference counterpart: the 2-D path of kernels/shared_mask_batched_triton_min_runtime.py
(KRN): the in-place kernel KRN:2289-2384, the compact-output kernel KRN:2473-2557, their
host entry `_prepacked_block_sparse_gemm_2d_from_active_blocks` (KRN:3498-3850), the bitmap
and compact wrappers (KRN:3853-4009), `_scatter_compact_to_dense_output` (KRN:3470-3495) and
the output-mask block list of `_get_cached_active_n_blocks_delta` (KRN:453-495).

Here every piece is one launch of libbsgemm: the GEMM kernels take the active output blocks as
a device list (each 64-column block is 64 / group-columns column tiles of the same kernels as
the 1-D path), the scatter and the mask-to-block list are small HIP kernels, and nothing
round-trips to the host except where the reference's Python API returns host-sized tensors.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from ._lib import Plan, check, load
from .runtime import (BLOCK_K, MAX_NBLK, _cu_count, _dtype_code, _pad_k, _packed_entry, _require_cuda,
                      _sort_active_blocks_asc, _stream_handle, _workspace, ctypes_byref, resolve_plan)

INDEX_BLOCK_OUT_META_SIZE = 64  # output-block width of the 2-D path (KRN:19)
BLOCK_N_OUT = INDEX_BLOCK_OUT_META_SIZE

# Compact-output buffers reused across calls, keyed like the reference's temp buffers
# (KRN:3112-3130): (prefix, shape, dtype, device).
_TEMP_BUFFERS: Dict[tuple, torch.Tensor] = {}


def _temp_buffer(prefix: str, shape: Tuple[int, ...], dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    key = (prefix, tuple(int(s) for s in shape), dtype, str(device))
    buf = _TEMP_BUFFERS.get(key)
    if buf is None:
        buf = torch.empty(shape, dtype=dtype, device=device)
        _TEMP_BUFFERS[key] = buf
    return buf


def _int32_dev(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    if t.device != dev:
        raise ValueError(f"block lists must be on {dev}, got {t.device}")
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def plan_2d(bt: int, n_dim: int, nn: int, nblk: int, na: int, device: torch.device, plan: Optional[Plan] = None,
            dense: bool = False) -> Plan:
    """A plan whose work-group covers at most one 64-column output block.  An explicit plan is
    kept (and rejected when wider).  Otherwise the tile is the one the 1-D path uses for the
    full N (the tuned table), or the library's when that one is wider than 64 columns, and the
    split-K factor fills the chip without a partial second round: floor(CUs / work-groups),
    at most 4 for 32- and 64-row tiles (their partials are large) and 8 otherwise, measured on
    down_proj B=16 and B=64 with 16-64 of 64 output blocks."""
    explicit = plan is not None and any(plan.as_tuple())
    pl = resolve_plan(bt, n_dim, nblk, na, device, plan, dense=dense)
    if pl.kind in (5, 6, 7):
        # variable-width column groups have no 2-D instantiation: the 16-column list-splitting
        # tile of the same rows instead
        if explicit:
            raise ValueError(f"2-D sparsity runs kinds 1-4; plan {pl.as_tuple()} is kind {pl.kind}")
        pl = resolve_plan(bt, n_dim, nblk, na, device, Plan(1, 16, 0, 0, pl.rows_per_group, 1), dense=dense,
                          lookup_plan=False)
    if pl.group_cols() > BLOCK_N_OUT:
        if explicit:
            raise ValueError(f"2-D sparsity needs a plan covering at most {BLOCK_N_OUT} columns per work-group; "
                             f"{pl.as_tuple()} covers {pl.group_cols()}")
        pl = resolve_plan(bt, n_dim, nblk, na, device, Plan(1, 16, 0, 0, pl.rows_per_group, pl.kind), dense=dense,
                          lookup_plan=False)
    if explicit and plan.split_k:
        return pl
    groups = max(1, nn) * (BLOCK_N_OUT // pl.group_cols()) * (-(-int(bt) // pl.rows_per_group))
    cap = 4 if pl.rows_per_group >= 32 else 8
    splitters = pl.waves_per_group if pl.kind == 1 else 1
    sk = max(1, min(cap, _cu_count(device) // groups, max(1, int(na) // (2 * splitters))))
    if pl.kind == 3:
        sk = 1
    return Plan(sk, pl.cols_per_wave, pl.waves_per_group, pl.depth, pl.rows_per_group, pl.kind)


def gemm_2d_packed(x2d: torch.Tensor, packed: torch.Tensor, n_dim: int, active_blocks: Optional[torch.Tensor],
                   n_blocks: torch.Tensor, y2d: torch.Tensor, *, num_active: Optional[int] = None,
                   num_active_dev: Optional[torch.Tensor] = None, num_n: Optional[int] = None,
                   num_n_dev: Optional[torch.Tensor] = None, compact: bool = False, plan: Optional[Plan] = None,
                   workspace_prefix: str = "gemm2d") -> Plan:
    """One 2-D block-sparse GEMM on packed weights (bsg_gemm_2d).

    x2d [bt, K]; `active_blocks` int32 K-block list (None: every K-block) with optional host
    length `num_active` and device count `num_active_dev`; `n_blocks` int32 list of active
    64-column output blocks (ascending), host length `num_n`, optional device count
    `num_n_dev`.  compact=False: y2d is [bt, N] and only the active blocks' columns are
    written; compact=True: y2d is [bt, num_n * 64], list entry i at columns 64i.."""
    lib = load()
    dev = _require_cuda(x2d, packed, y2d)
    code = _dtype_code(x2d)
    bt, k_dim = x2d.shape
    x2d = _pad_k(x2d)
    nblk = int(packed.shape[0])
    if (k_dim + BLOCK_K - 1) // BLOCK_K != nblk:
        raise ValueError(f"x has K={k_dim} but the packed weight has {nblk} K-blocks")
    nnb = (int(n_dim) + BLOCK_N_OUT - 1) // BLOCK_N_OUT
    nn = int(n_blocks.numel() if num_n is None else num_n)
    if nn < 0 or nn > nnb or nn > int(n_blocks.numel()):
        raise ValueError(f"{nn} active output blocks for N={n_dim} ({nnb} blocks, list of {n_blocks.numel()})")
    width = nn * BLOCK_N_OUT if compact else int(n_dim)
    if y2d.shape[0] != bt or y2d.shape[1] < width or y2d.stride(1) != 1 or (not compact and y2d.shape[1] != n_dim):
        raise ValueError(f"y must be [bt, {width}] with unit column stride, got {tuple(y2d.shape)}")
    if bt == 0 or nn == 0:
        return Plan()
    nb = _int32_dev(n_blocks, dev)
    if active_blocks is not None:
        ab = _int32_dev(active_blocks, dev)
        na = int(ab.numel() if num_active is None else num_active)
        if na > MAX_NBLK or na > int(ab.numel()):
            raise ValueError(f"{na} active K-blocks (list of {ab.numel()}, at most {MAX_NBLK})")
    else:
        ab, na = None, nblk
    pl = plan_2d(bt, int(n_dim), nn, nblk, na, dev, plan, dense=active_blocks is None)
    ws_bytes = int(lib.bsg_gemm_workspace_bytes(bt, n_dim, ctypes_byref(pl)))
    ws_ptr = (_workspace(workspace_prefix, dev, ws_bytes, (bt, n_dim) + pl.as_tuple()).data_ptr()
              if ws_bytes > 0 else None)
    with torch.cuda.device(dev):
        rc = lib.bsg_gemm_2d(x2d.data_ptr(), x2d.stride(0), bt, x2d.shape[1], packed.data_ptr(), n_dim,
                             ab.data_ptr() if ab is not None and na > 0 else None, na if ab is not None else 0,
                             num_active_dev.data_ptr() if num_active_dev is not None else None,
                             nb.data_ptr(), nn, num_n_dev.data_ptr() if num_n_dev is not None else None,
                             1 if compact else 0, y2d.data_ptr(), y2d.stride(0), code, ws_ptr, ws_bytes,
                             ctypes_byref(pl), _stream_handle(dev))
    check(rc)
    return pl


def scatter_nblocks(compact2d: torch.Tensor, n_blocks: torch.Tensor, out2d: torch.Tensor, *,
                    num_n: Optional[int] = None, num_n_dev: Optional[torch.Tensor] = None) -> None:
    """out2d[:, 64 b_i + c] = compact2d[:, 64 i + c] for the active blocks b_i (bsg_scatter_nblocks)."""
    lib = load()
    dev = _require_cuda(compact2d, out2d)
    if compact2d.dtype != out2d.dtype or compact2d.element_size() != 2:
        raise TypeError(f"scatter copies 16-bit elements of one dtype ({compact2d.dtype} -> {out2d.dtype})")
    if compact2d.stride(1) != 1 or out2d.stride(1) != 1 or compact2d.shape[0] != out2d.shape[0]:
        raise ValueError("compact and out must be [bt, *] with unit column stride")
    nb = _int32_dev(n_blocks, dev)
    nn = int(nb.numel() if num_n is None else num_n)
    if nn < 0 or nn > int(nb.numel()) or compact2d.shape[1] < nn * BLOCK_N_OUT:
        raise ValueError(f"{nn} blocks: list of {nb.numel()}, compact width {compact2d.shape[1]}")
    with torch.cuda.device(dev):
        rc = lib.bsg_scatter_nblocks(compact2d.data_ptr(), compact2d.stride(0), compact2d.shape[0], nb.data_ptr(),
                                     nn, num_n_dev.data_ptr() if num_n_dev is not None else None, out2d.shape[1],
                                     out2d.data_ptr(), out2d.stride(0), _stream_handle(dev))
    check(rc)


def nmask_blocks(mask_u8: torch.Tensor, n_dim: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Active 64-column blocks of an element mask over N, on the device (bsg_nmask_blocks):
    returns (blocks int32[ceil(N/64)], count int32[1]); blocks[:count] ascending."""
    lib = load()
    dev = _require_cuda(mask_u8)
    if mask_u8.dtype not in (torch.uint8, torch.bool, torch.int8):
        raise TypeError(f"mask must be uint8/bool, got {mask_u8.dtype}")
    m = mask_u8.reshape(-1).contiguous()
    n = int(m.numel() if n_dim is None else n_dim)
    if n > int(m.numel()):
        raise ValueError(f"mask holds {m.numel()} entries, fewer than N={n}")
    blocks = torch.empty(max(1, (n + BLOCK_N_OUT - 1) // BLOCK_N_OUT), dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        check(lib.bsg_nmask_blocks(m.data_ptr(), n, blocks.data_ptr(), count.data_ptr(), _stream_handle(dev)))
    return blocks, count


# ---------------------------------------------------------------------------------------
# The reference's Python entry points (same names, arguments and return values)


def _get_cached_active_n_blocks_delta(mask_u8: torch.Tensor, prefix: str, block_size: int) -> torch.Tensor:
    """Sorted int32 ids of the `block_size`-column blocks with any nonzero mask entry
    (KRN:453-495).  The reference keeps per-prefix delta state to update the list
    incrementally; here the device kernel recomputes it from the mask every call (one launch
    plus the count read the returned length needs), so `prefix` only names the call site."""
    if int(block_size) != BLOCK_N_OUT:
        raise ValueError(f"block_size must be {BLOCK_N_OUT} (the output-block width), got {block_size}")
    blocks, count = nmask_blocks(mask_u8)
    return blocks[: int(count.item())].clone()


def _scatter_compact_to_dense_output(compact_out: torch.Tensor, active_n_blocks: torch.Tensor, block_n: int,
                                     out_dense: torch.Tensor) -> None:
    """Scatter compact [B, S, num_active * block_n] output to the dense N axis (KRN:3470-3495)."""
    if int(block_n) != BLOCK_N_OUT:
        raise ValueError(f"block_n must be {BLOCK_N_OUT}, got {block_n}")
    if int(active_n_blocks.numel()) <= 0:
        return
    bsz, seqlen, cw = compact_out.shape
    bt = bsz * seqlen
    if not out_dense.is_contiguous():
        raise ValueError("out_dense must be contiguous")
    nn = min(int(active_n_blocks.numel()), cw // BLOCK_N_OUT)
    scatter_nblocks(compact_out.reshape(bt, cw), active_n_blocks, out_dense.view(bt, out_dense.shape[-1]), num_n=nn)


def _prepacked_block_sparse_gemm_2d_from_active_blocks(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_k_blocks: torch.Tensor,
    active_n_blocks: Optional[torch.Tensor],
    out: torch.Tensor,
    cache_prefix: str = "gemm2d",
    proj_tag: str = "",
    sort_active_k_blocks: bool = True,
    sort_active_n_blocks: bool = True,
    zero_fill_out: bool = False,
    compact_output: bool = False,
    scatter_compact_to_dense: bool = False,
    active_n_mask_u8: Optional[torch.Tensor] = None,
    active_k_blocks_limit: Optional[int] = None,
    active_n_blocks_limit: Optional[int] = None,
) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    """Y over active K-blocks, computed only in the active 64-column output blocks
    (KRN:3498-3850).  Returns (compact output [B, S, num_n * 64] or None, active output block
    ids).  `active_n_blocks` None: from `active_n_mask_u8`, else every block.  In place, the
    inactive columns of `out` are left as they are unless `zero_fill_out`.  `proj_tag` only
    chose tuned Triton launch metadata there and is accepted for compatibility.  N is the
    weight's output width (the reference took it from `out`, which for compact callers is the
    compact width)."""
    if x.dim() != 3:
        raise ValueError(f"x must be [B, S, K], got {tuple(x.shape)}")
    bsz, seqlen, m_dim = x.shape
    n_dim = int(weight.shape[0])
    dev = x.device
    num_k = int(active_k_blocks.numel()) if active_k_blocks_limit is None else int(active_k_blocks_limit)
    num_k = min(num_k, int(active_k_blocks.numel()))
    if num_k <= 0:
        out.zero_()
        return None, torch.empty((0,), device=dev, dtype=torch.int32)
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    kb = _int32_dev(active_k_blocks, dev)[:num_k].contiguous()
    if sort_active_k_blocks:
        kb = _sort_active_blocks_asc(kb)
    if active_n_blocks is None and active_n_mask_u8 is not None:
        active_n_blocks = _get_cached_active_n_blocks_delta(active_n_mask_u8, f"{cache_prefix}_nout", BLOCK_N_OUT)
    if active_n_blocks is None:
        active_n_blocks = torch.arange((n_dim + BLOCK_N_OUT - 1) // BLOCK_N_OUT, device=dev, dtype=torch.int32)
    nb = _int32_dev(active_n_blocks, dev)
    if sort_active_n_blocks:
        nb = _sort_active_blocks_asc(nb)
    num_n = int(nb.numel()) if active_n_blocks_limit is None else min(int(active_n_blocks_limit), int(nb.numel()))
    if num_n <= 0:
        out.zero_()
        return None, nb
    nb_ret = nb[:num_n].contiguous()
    bt = bsz * seqlen
    x2d = x.reshape(bt, m_dim)
    if compact_output:
        width = num_n * BLOCK_N_OUT
        y_c = _temp_buffer(f"{cache_prefix}_compact2d_out", (bt, width), x.dtype, dev)
        gemm_2d_packed(x2d, entry.packed, n_dim, kb, nb_ret, y_c, compact=True,
                       workspace_prefix=f"{cache_prefix}_ws2d")
        y_c3 = y_c.view(bsz, seqlen, width)
        if scatter_compact_to_dense:
            if zero_fill_out:
                out.zero_()
            _scatter_compact_to_dense_output(y_c3, nb_ret, BLOCK_N_OUT, out)
        return y_c3, nb_ret
    if out.shape[-1] != n_dim or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous [B, S, N={n_dim}], got {tuple(out.shape)}")
    if zero_fill_out:
        out.zero_()
    gemm_2d_packed(x2d, entry.packed, n_dim, kb, nb_ret, out.view(bt, n_dim), workspace_prefix=f"{cache_prefix}_ws2d")
    return None, nb_ret


def _prepacked_block_sparse_gemm_2d_bitmap_from_active_blocks(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_k_blocks: torch.Tensor,
    active_n_blocks: Optional[torch.Tensor],
    out: torch.Tensor,
    cache_prefix: str = "gemm2d_bmp",
    sort_active_n_blocks: bool = True,
    zero_fill_out: bool = False,
    active_k_blocks_limit: Optional[int] = None,
    active_n_blocks_limit: Optional[int] = None,
) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    """The reference's K-bitmap variant of the 2-D path (KRN:3853-3966).  The same result
    comes from the list kernel here (the K-blocks are walked in ascending order either way)."""
    return _prepacked_block_sparse_gemm_2d_from_active_blocks(
        x, weight, active_k_blocks, active_n_blocks, out, cache_prefix=cache_prefix, sort_active_k_blocks=True,
        sort_active_n_blocks=sort_active_n_blocks, zero_fill_out=zero_fill_out,
        active_k_blocks_limit=active_k_blocks_limit, active_n_blocks_limit=active_n_blocks_limit)


def _prepacked_block_sparse_gemm_2d_compact_from_active_blocks(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_k_blocks: torch.Tensor,
    active_n_blocks: Optional[torch.Tensor],
    cache_prefix: str = "gemm2d_compact",
    proj_tag: str = "",
    sort_active_k_blocks: bool = True,
    sort_active_n_blocks: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Compact output of the active output blocks plus their ids (KRN:3969-4009); an empty or
    missing output list gives a [B, S, 0] result."""
    bsz, seqlen, _ = x.shape
    num_n = int(active_n_blocks.numel()) if active_n_blocks is not None else 0
    if num_n <= 0:
        return (torch.empty((bsz, seqlen, 0), device=x.device, dtype=x.dtype),
                torch.empty((0,), device=x.device, dtype=torch.int32))
    out_compact = torch.empty((bsz, seqlen, num_n * BLOCK_N_OUT), device=x.device, dtype=x.dtype)
    compact, blocks = _prepacked_block_sparse_gemm_2d_from_active_blocks(
        x, weight, active_k_blocks, active_n_blocks, out_compact, cache_prefix=cache_prefix, proj_tag=proj_tag,
        sort_active_k_blocks=sort_active_k_blocks, sort_active_n_blocks=sort_active_n_blocks,
        compact_output=True)
    if compact is None:
        return out_compact, blocks
    out_compact.copy_(compact)
    return out_compact, blocks
