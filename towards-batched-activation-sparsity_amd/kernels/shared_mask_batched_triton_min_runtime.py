"""Drop-in module for `kernels.shared_mask_batched_triton_min_runtime`.

The reference's drivers import their GEMM entry points from this module path
(scripts/bench_perstep_actual_kernel_speedup.py:29-35, scripts/profile_kernel_configs.py:23-31,
scripts/bench_roundrobin_e2e_decode.py:27-35).  Putting the directory that holds this package
first on sys.path makes those imports resolve here: every name below is the HIP/CDNA4
implementation from bsa_mi355x (no Triton is involved; the module keeps the reference's file
name only so callers need no edits).
"""
from bsa_mi355x.runtime import (  # noqa: F401
    INDEX_BLOCK_META_SIZE,
    _WEIGHT_PREPACK_CACHE,
    _WORKSPACE_CACHE,
    _build_active_k_bitmap,
    _get_prepacked_weight_block_major,
    _prepacked_block_sparse_gemm_from_active_blocks,
    _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload,
    _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk,
    _prepacked_block_sparse_gemm_from_active_blocks_splitk,
    _sort_active_blocks_asc,
    prepacked_block_sparse_gemm_batched_kernel,
    prepacked_block_sparse_gemm_bitmap_preload_batched_kernel,
)
from bsa_mi355x.select import _select_active_blocks_l1  # noqa: F401
from bsa_mi355x.sparse2d import (  # noqa: F401
    INDEX_BLOCK_OUT_META_SIZE,
    _get_cached_active_n_blocks_delta,
    _prepacked_block_sparse_gemm_2d_bitmap_from_active_blocks,
    _prepacked_block_sparse_gemm_2d_compact_from_active_blocks,
    _prepacked_block_sparse_gemm_2d_from_active_blocks,
    _scatter_compact_to_dense_output,
)


def __getattr__(name: str):
    # _PREPACK_AUTOTUNE_CONFIGS is built on first use from the library's kernel table.
    if name == "_PREPACK_AUTOTUNE_CONFIGS":
        from bsa_mi355x import runtime

        return runtime._PREPACK_AUTOTUNE_CONFIGS
    raise AttributeError(name)
