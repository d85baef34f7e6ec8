"""bsa_mi355x — MI355X (gfx950) batch-shared 64-channel block-sparse activation GEMM.

    Y[B, N] = X[B, active K-blocks] · W[active K-blocks, N]

with one active-block mask shared by the whole decode batch.  Kernels are hand-written HIP
for CDNA4 (csrc/bsgemm.hip) behind a C ABI (include/bsgemm.h); this package is the host
layer that mirrors the reference's Python entry points
(kernels/shared_mask_batched_triton_min_runtime.py).
"""
from ._lib import BLOCK_K, MAX_NBLK, BsgArgError, BsgDtypeError, BsgError, BsgUnsupported, Plan, load
from .autotune import set_autotune
from .runtime import (INDEX_BLOCK_META_SIZE, TiledPackedWeight, TileConfig, _build_active_k_bitmap, _get_prepacked_weight_block_major,
                      _prepacked_block_sparse_gemm_from_active_blocks,
                      _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload,
                      _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk,
                      _prepacked_block_sparse_gemm_from_active_blocks_splitk, _sort_active_blocks_asc, active_bytes,
                      dense_gemm, gemm_packed, kernel_tiles, make_plan, n_keep_for_density, nblk_of, pack_weight,
                      prepacked_block_sparse_gemm_batched_kernel,
                      prepacked_block_sparse_gemm_bitmap_preload_batched_kernel, release_prepacked_weights,
                      resolve_plan)
from .select import (_energy_expanded_active_blocks, _select_active_blocks, _select_active_blocks_l1,
                     _topk_energy_ratio, select_sparse_gemm, select_topk, select_topk_l1)
from .sparse2d import (INDEX_BLOCK_OUT_META_SIZE, _get_cached_active_n_blocks_delta,
                       _prepacked_block_sparse_gemm_2d_bitmap_from_active_blocks,
                       _prepacked_block_sparse_gemm_2d_compact_from_active_blocks,
                       _prepacked_block_sparse_gemm_2d_from_active_blocks, _scatter_compact_to_dense_output,
                       gemm_2d_packed, nmask_blocks, scatter_nblocks)

__all__ = [
    "BLOCK_K", "MAX_NBLK", "INDEX_BLOCK_META_SIZE", "Plan", "TileConfig", "TiledPackedWeight", "load",
    "BsgError", "BsgArgError", "BsgDtypeError", "BsgUnsupported", "set_autotune",
    "_build_active_k_bitmap", "_get_prepacked_weight_block_major", "_sort_active_blocks_asc",
    "_prepacked_block_sparse_gemm_from_active_blocks",
    "_prepacked_block_sparse_gemm_from_active_blocks_splitk",
    "_prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload",
    "_prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk",
    "prepacked_block_sparse_gemm_batched_kernel", "prepacked_block_sparse_gemm_bitmap_preload_batched_kernel",
    "dense_gemm", "gemm_packed", "pack_weight", "make_plan", "resolve_plan", "kernel_tiles",
    "release_prepacked_weights", "n_keep_for_density", "active_bytes", "nblk_of",
    "select_topk_l1", "select_topk", "select_sparse_gemm", "_select_active_blocks_l1", "_select_active_blocks",
    "_topk_energy_ratio", "_energy_expanded_active_blocks",
    "INDEX_BLOCK_OUT_META_SIZE", "_prepacked_block_sparse_gemm_2d_from_active_blocks",
    "_prepacked_block_sparse_gemm_2d_bitmap_from_active_blocks",
    "_prepacked_block_sparse_gemm_2d_compact_from_active_blocks", "_scatter_compact_to_dense_output",
    "_get_cached_active_n_blocks_delta", "gemm_2d_packed", "scatter_nblocks", "nmask_blocks",
]
