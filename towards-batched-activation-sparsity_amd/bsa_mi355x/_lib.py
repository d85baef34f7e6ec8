"""ctypes binding of libbsgemm.so (C ABI declared in include/bsgemm.h).

The library is loaded after torch so that its libamdhip64.so.7 dependency resolves to the
HIP runtime torch already mapped (same SONAME): device pointers and hipStream_t handles
taken from torch tensors and streams are then valid inside the library.
There is no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# BSA_MI355X_LIB=timeline selects the phase-timeline profiling build (libbsgemm_timeline.so,
# same ABI, kernels that record per-work-group stamps); the default is the shipped library.
LIB_PATH = os.path.join(_HERE, "libbsgemm_timeline.so" if os.environ.get("BSA_MI355X_LIB") == "timeline"
                        else "libbsgemm.so")

BSG_OK = 0
BSG_ERR_ARG = -1
BSG_ERR_DTYPE = -2
BSG_ERR_WORKSPACE = -3
BSG_ERR_ALIGN = -4
BSG_ERR_UNSUPPORTED = -5
BSG_ERR_HIP = -100

BSG_F16 = 0
BSG_BF16 = 1
BLOCK_K = 64
MAX_NBLK = 2048
NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # BSG_NOALLOC_SCRATCH_BYTES


class BsgError(RuntimeError):
    """A libbsgemm call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libbsgemm status {status}: {message}")
        self.status = status


class BsgArgError(BsgError, ValueError):
    pass


class BsgDtypeError(BsgError, TypeError):
    pass


class BsgUnsupported(BsgError, NotImplementedError):
    pass


class Plan(ctypes.Structure):
    """Mirror of `bsg_plan`; zero fields are resolved by the library."""

    _fields_ = [
        ("split_k", ctypes.c_int32),
        ("cols_per_wave", ctypes.c_int32),
        ("waves_per_group", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("rows_per_group", ctypes.c_int32),
        ("kind", ctypes.c_int32),
    ]

    def as_tuple(self):
        return (self.split_k, self.cols_per_wave, self.waves_per_group, self.depth, self.rows_per_group, self.kind)

    def group_cols(self) -> int:
        """Output columns one work-group covers: waves split columns in kind 2, column groups
        x channel halves in kind 4, the block list in kinds 1 and 3."""
        if self.kind == 2:
            return self.cols_per_wave * self.waves_per_group
        if self.kind == 4:
            return self.cols_per_wave * (self.waves_per_group // 2)
        return self.cols_per_wave

    def __repr__(self) -> str:
        return ("Plan(split_k=%d, cols_per_wave=%d, waves_per_group=%d, depth=%d, rows_per_group=%d, kind=%d)"
                % self.as_tuple())


BSG_SCORE_L1, BSG_SCORE_L2_MEAN, BSG_SCORE_ENERGY = 0, 1, 2


class SelectOpts(ctypes.Structure):
    """Mirror of `bsg_select_opts` (pointers are device addresses or None)."""

    _fields_ = [
        ("score", ctypes.c_int32),
        ("energy_keep", ctypes.c_float),
        ("block_prior", ctypes.c_void_p),
        ("prior_alpha", ctypes.c_float),
        ("prior_eps", ctypes.c_float),
        ("channel_scale", ctypes.c_void_p),
        ("ratio_out", ctypes.c_void_p),
    ]


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_pplan = ctypes.POINTER(Plan)

# name -> (restype, argtypes); every function declared in include/bsgemm.h
SIGNATURES = {
    "bsg_version": (ctypes.c_char_p, []),
    "bsg_last_error": (ctypes.c_char_p, []),
    "bsg_packed_bytes": (_i64, [_i64, _i64, _int]),
    "bsg_pack_weight": (_int, [_vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp]),
    "bsg_plan_resolve": (_int, [_i64, _i64, _i32, _i32, _i32, _pplan]),
    "bsg_gemm_workspace_bytes": (_i64, [_i64, _i64, _pplan]),
    "bsg_workspace_init": (_int, [_vp, _i64, _vp]),
    "bsg_gemm": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _i64, _int, _vp, _i64, _pplan, _vp]),
    "bsg_gemm_sorted": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _i64, _int, _vp, _i64, _pplan,
                               _vp]),
    "bsg_gemm_bitmap": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _i64, _int, _vp, _i64, _pplan, _vp]),
    "bsg_gemm_dense": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _int, _vp, _i64, _pplan, _vp]),
    "bsg_gemm_2d": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _i32, _vp, _int, _vp, _i64, _int,
                           _vp, _i64, _pplan, _vp]),
    "bsg_scatter_nblocks": (_int, [_vp, _i64, _i64, _vp, _i32, _vp, _i64, _vp, _i64, _vp]),
    "bsg_nmask_blocks": (_int, [_vp, _i64, _vp, _vp, _vp]),
    "bsg_select_workspace_bytes": (_i64, [_i64]),
    "bsg_select_topk_l1": (_int, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _int, _vp, _i64, _vp]),
    "bsg_select_topk": (_int, [_vp, _i64, _i64, _i64, _i32, ctypes.POINTER(SelectOpts), _vp, _vp, _int, _vp,
                               _i64, _vp]),
    "bsg_select_gemm": (_int, [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _int, _vp, _i64,
                               _pplan, _vp]),
    "bsg_select_gemm_rule": (_int, [_vp, _i64, _i64, _i64, _i32, ctypes.POINTER(SelectOpts), _vp, _i64, _vp, _vp,
                                    _vp, _i64, _int, _vp, _i64, _pplan, _vp]),
    "bsg_select_gemm_noalloc": (_int, [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _int,
                                       _pplan, _vp]),
    "bsg_read_calibrate": (_int, [_vp, _i64, _vp, _vp]),
    # include/bsgemm_timeline.h
    "bsg_timeline_attach": (_int, [_vp, _i64, _i64]),
    "bsg_timeline_clock_khz": (_i64, []),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load (once) and return the ctypes library handle."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (maps torch's libamdhip64.so.7 first)

        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library not built: {LIB_PATH} is missing. Build it with "
                "`python towards-batched-activation-sparsity_amd/build.py` or __graft_entry__.build().")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    return load().bsg_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    """Raise the Python exception matching a libbsgemm status."""
    if status == BSG_OK:
        return
    msg = last_error()
    if status in (BSG_ERR_ARG, BSG_ERR_ALIGN):
        raise BsgArgError(status, msg)
    if status == BSG_ERR_DTYPE:
        raise BsgDtypeError(status, msg)
    if status == BSG_ERR_UNSUPPORTED:
        raise BsgUnsupported(status, msg)
    raise BsgError(status, msg)
