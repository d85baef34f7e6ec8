"""Host layer of the MI355X block-sparse GEMM, mirroring the reference's Python interface.

The public names, argument meanings, in-place `out` convention and `num_active == 0 ->
out.zero_()` behaviour follow kernels/shared_mask_batched_triton_min_runtime.py (cited per
function).  Every GEMM is one launch of the HIP kernel family in csrc/bsgemm.hip through the
C ABI (include/bsgemm.h); torch only supplies device memory, streams and views.

Differences from the reference that are deliberate:
  * A non-contiguous `out` raises ValueError (the reference silently writes a temporary,
    KRN:1029-1032, 1114-1117, 3199-3202).
  * The packed-weight cache entry is tied to the weight tensor (weakref + version counter),
    so a freed-and-reused address or an in-place weight update triggers a re-pack instead of
    returning stale data (the reference keys on data_ptr only, KRN:3134-3150).
  * Split-K is always the deterministic in-kernel reduction (no atomic accumulation path).
"""
from __future__ import annotations

import math
import weakref
from typing import Dict, Optional, Sequence

import torch

from . import _lib
from ._lib import BLOCK_K, MAX_NBLK, Plan, check, load

INDEX_BLOCK_META_SIZE = BLOCK_K  # KRN:17

_DTYPES = {torch.float16: _lib.BSG_F16, torch.bfloat16: _lib.BSG_BF16}

# Cache dicts with hit/miss counters, like the reference's module-level caches (KRN:74-120).
_WEIGHT_PREPACK_CACHE: Dict[str, dict] = {"gemm": {}, "hits": 0, "misses": 0}
_WORKSPACE_CACHE: Dict[str, dict] = {"bufs": {}, "hits": 0, "misses": 0}

_CU_COUNT: Dict[int, int] = {}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"block-sparse GEMM supports float16/bfloat16, got {t.dtype}") from None


def _stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def _cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _CU_COUNT[idx]


def _require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError("block-sparse GEMM tensors must live on a ROCm (cuda) device")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got {t.device}")
    return dev


# ---------------------------------------------------------------------------------------
# Weight packing (KRN:3133-3163)


class _PackEntry:
    __slots__ = ("packed", "n", "k", "nblk", "npad", "ref", "version")

    def __init__(self, packed, n, k, ref, version):
        self.packed = packed
        self.n = n
        self.k = k
        self.nblk = (k + BLOCK_K - 1) // BLOCK_K
        self.npad = (n + 15) // 16 * 16
        self.ref = ref
        self.version = version


def pack_weight(weight: torch.Tensor, layout: str = "nk") -> torch.Tensor:
    """Pack a weight into the tiled K-major layout; returns a tensor [nblk, Np/16, 1024].

    layout "nk": weight is nn.Linear's [N, K] (reference input, KRN:3135);
    layout "kn": weight is stored [K, N] (the reference's packed row order before the
    [nblk, 64, N] view).
    """
    lib = load()
    dev = _require_cuda(weight)
    code = _dtype_code(weight)
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D, got {tuple(weight.shape)}")
    if layout == "nk":
        n, k = weight.shape
        sn, sk = weight.stride(0), weight.stride(1)
    elif layout == "kn":
        k, n = weight.shape
        sk, sn = weight.stride(0), weight.stride(1)
    else:
        raise ValueError(f"layout must be 'nk' or 'kn', got {layout!r}")
    nbytes = int(lib.bsg_packed_bytes(n, k, code))
    if nbytes <= 0:
        raise ValueError(f"cannot pack weight of shape {tuple(weight.shape)}")
    nblk = (k + BLOCK_K - 1) // BLOCK_K
    ntile = (n + 15) // 16
    packed = torch.empty((nblk, ntile, 1024), dtype=weight.dtype, device=dev)
    with torch.cuda.device(dev):
        check(lib.bsg_pack_weight(weight.data_ptr(), n, k, sn, sk, code, packed.data_ptr(), nbytes,
                                  _stream_handle(dev)))
    return packed


def _packed_entry(weight: torch.Tensor, block_k: int, cache_prefix: str) -> _PackEntry:
    if int(block_k) != BLOCK_K:
        raise ValueError(f"block_k must be {BLOCK_K} (the kernels' K-block), got {block_k}")
    cache = _WEIGHT_PREPACK_CACHE.setdefault(cache_prefix, {})
    n_dim, m_dim = weight.shape
    key = (cache_prefix, int(weight.data_ptr()), str(weight.device), str(weight.dtype), int(n_dim), int(m_dim),
           int(weight.stride(0)), int(weight.stride(1)), int(block_k))
    entry = cache.get(key)
    if entry is not None:
        owner = entry.ref()
        if owner is not None and owner._version == entry.version:
            _WEIGHT_PREPACK_CACHE["hits"] += 1
            return entry
        del cache[key]
    _WEIGHT_PREPACK_CACHE["misses"] += 1
    packed = pack_weight(weight, "nk")
    entry = _PackEntry(packed, int(n_dim), int(m_dim), weakref.ref(weight), weight._version)
    cache[key] = entry
    return entry


class TiledPackedWeight(torch.Tensor):
    """What `_get_prepacked_weight_block_major` returns: the cached packed weight, sharing its
    storage, in this build's MFMA tile order [nblk, Np/16, 1024] (element (j, k, n) at
    [j, n // 16, (k // 32) * 512 + ((k % 32) // 8) * 128 + (n % 16) * 8 + k % 8], Np = N
    rounded up to 16), not the reference's [nblk, 64, N] (KRN:3162).  The reference's drivers
    only call the function to warm the cache (BPS:160, PKC:116, RRD:321-324); code that sliced
    the result as the reference layout would read the wrong elements, so Python indexing
    raises.  `block_major(n)` returns the reference layout (a copy)."""

    def __getitem__(self, item):
        raise TypeError("the packed weight is in the MFMA tile order [nblk, Np/16, 1024], not [nblk, 64, N]; "
                        "use .block_major(N) for the reference layout")

    def block_major(self, n: int) -> torch.Tensor:
        """The reference's [nblk, 64, n] block-major packing (KRN:3152-3162), as a new tensor."""
        w = self.as_subclass(torch.Tensor)
        nblk, t16, _ = w.shape
        # [j, t, h, g, c, e] -> [j, h, g, e, t, c]: k = 32h + 8g + e, n = 16t + c
        w6 = w.reshape(nblk, t16, 2, 4, 16, 8).permute(0, 2, 3, 5, 1, 4)
        return w6.reshape(nblk, BLOCK_K, t16 * 16)[:, :, : int(n)].contiguous()

    def __repr__(self) -> str:
        return f"TiledPackedWeight(shape={tuple(self.shape)}, dtype={self.dtype}, device={self.device})"


def _get_prepacked_weight_block_major(weight: torch.Tensor, block_k: int, cache_prefix: str = "gemm") -> torch.Tensor:
    """Packed weight for nn.Linear `weight` [N, K], cached per prefix (KRN:3133-3163), as a
    TiledPackedWeight view of the cache entry."""
    return _packed_entry(weight, block_k, cache_prefix).packed.as_subclass(TiledPackedWeight)


def release_prepacked_weights(cache_prefix: Optional[str] = None) -> None:
    """Drop cached packed weights (all prefixes, or one), and the prepared drop-in calls that
    hold them."""
    for name, cache in list(_WEIGHT_PREPACK_CACHE.items()):
        if isinstance(cache, dict) and (cache_prefix is None or name == cache_prefix):
            cache.clear()
    for key in [k for k in _PREPARED if cache_prefix is None or k[0] == cache_prefix]:
        del _PREPARED[key]
    for hook in _FORGET_HOOKS:
        hook()


# ---------------------------------------------------------------------------------------
# Plans, workspaces


def _pow2_at_least(v: int, lo: int, hi: int) -> int:
    p = lo
    while p < v and p < hi:
        p <<= 1
    return p


def make_plan(num_split_k: Optional[int] = None, tile_b: Optional[int] = None, tile_n: Optional[int] = None,
              tile_warps: Optional[int] = None, tile_stages: Optional[int] = None, bt: int = 0) -> Plan:
    """Map the reference's split-K factor and Triton tile (BLOCK_B, BLOCK_N, num_warps,
    num_stages) (KRN:1296-1299, 1350-1361) onto a bsg_plan; None means automatic.

    A batch tile smaller than the batch would make every row group re-stream the weight, so
    BLOCK_B is raised to cover min(bt, 64) rows."""
    p = Plan()
    p.split_k = int(num_split_k) if num_split_k else 0
    p.rows_per_group = _pow2_at_least(max(int(tile_b), min(int(bt), 64)), 16, 64) if tile_b else 0
    p.cols_per_wave = _pow2_at_least(int(tile_n), 16, 128) if tile_n else 0
    p.waves_per_group = _pow2_at_least(int(tile_warps), 1, 8) if tile_warps else 0
    p.depth = _pow2_at_least(int(tile_stages), 1, 8) if tile_stages else 0
    return p


# The library's plan resolution is a pure function of (problem, CU count, requested plan); its
# answers are kept so that an eager call pays one dictionary lookup instead of a library call.
_RESOLVED: dict = {}


def resolve_plan(bt: int, n: int, nblk: int, na: int, device: torch.device, plan: Optional[Plan] = None,
                 dense: bool = False, lookup_plan: bool = True, select: bool = False) -> Plan:
    """Resolve a (partial) plan for a problem.  With no plan (or an all-zero one) the tuned
    table (tuning.lookup; select=True: the entries timed as selection + GEMM first) is consulted
    first; remaining zero fields are filled by the library's heuristics; tile fields that name a
    kernel that is not instantiated fall back to automatic (the split-K factor is kept)."""
    lib = load()
    if lookup_plan and (plan is None or not any(plan.as_tuple())):
        from . import tuning

        tuned = tuning.lookup(bt, n, nblk, na, dense=dense, select=select)
        if tuned is not None:
            plan = tuned
    req = plan.as_tuple() if plan is not None else (0, 0, 0, 0, 0, 0)
    key = (int(bt), int(n), int(nblk), int(na), _cu_count(device), req)
    hit = _RESOLVED.get(key)
    if hit is not None:
        return Plan(*hit)
    out = Plan(*req)
    rc = lib.bsg_plan_resolve(bt, n, nblk, na, key[4], ctypes_byref(out))
    if rc == _lib.BSG_ERR_UNSUPPORTED:
        out = Plan(req[0], 0, 0, 0, 0, 0)
        rc = lib.bsg_plan_resolve(bt, n, nblk, na, key[4], ctypes_byref(out))
    check(rc)
    _RESOLVED[key] = out.as_tuple()
    return out


def ctypes_byref(p: Plan):
    import ctypes

    return ctypes.byref(p)


def _workspace(prefix: str, device: torch.device, nbytes: int, layout: tuple = ()) -> torch.Tensor:
    """Zero-initialised workspace cached by (prefix, device, size, layout) like the reference's
    split-K partial buffers (KRN:3099-3109).  The GEMM leaves its counters at zero, so a
    cached workspace is reusable without clearing; `layout` (problem shape and plan) keeps
    launches whose counter regions end at different offsets on separate buffers.  Two GEMMs in
    flight on different streams must not share a prefix."""
    cache = _WORKSPACE_CACHE["bufs"]
    key = (prefix, str(device), int(nbytes), tuple(layout))
    buf = cache.get(key)
    if buf is None:
        _WORKSPACE_CACHE["misses"] += 1
        buf = torch.zeros(int(nbytes), dtype=torch.uint8, device=device)
        cache[key] = buf
    else:
        _WORKSPACE_CACHE["hits"] += 1
    return buf


# ---------------------------------------------------------------------------------------
# GEMM entry points


class _KernelHandle:
    """Stands in for a Triton autotuned kernel object: `best_config` reports the tile of the
    last launch (scripts/profile_kernel_configs.py:135 reads it): the tuned table's plan for a
    tabulated problem, the first-call tuned winner for any other key (bsa_mi355x.autotune), or
    the explicit plan the call named."""

    def __init__(self, name: str):
        self.__name__ = name
        self.last_plan: Optional[Plan] = None

    @property
    def best_config(self):
        p = self.last_plan
        if p is None:
            return None
        return TileConfig({"BLOCK_B": p.rows_per_group, "BLOCK_N": p.group_cols()}, num_warps=p.waves_per_group,
                          num_stages=p.depth, split_k=p.split_k, kind=p.kind)


class TileConfig:
    """Duck-types triton.Config (.kwargs["BLOCK_B"/"BLOCK_N"], .num_warps, .num_stages) for
    the drivers that enumerate tiles (scripts/profile_kernel_configs.py:70-83)."""

    def __init__(self, kwargs: dict, num_warps: int, num_stages: int, split_k: int = 0, kind: int = 0):
        self.kwargs = dict(kwargs)
        self.num_warps = int(num_warps)
        self.num_stages = int(num_stages)
        self.split_k = int(split_k)
        self.kind = int(kind)

    def __repr__(self) -> str:
        return (f"TileConfig(BLOCK_B={self.kwargs['BLOCK_B']}, BLOCK_N={self.kwargs['BLOCK_N']}, "
                f"num_warps={self.num_warps}, num_stages={self.num_stages})")


prepacked_block_sparse_gemm_batched_kernel = _KernelHandle("prepacked_block_sparse_gemm_batched_kernel")
prepacked_block_sparse_gemm_bitmap_preload_batched_kernel = _KernelHandle(
    "prepacked_block_sparse_gemm_bitmap_preload_batched_kernel")


def _views(x: torch.Tensor, out: torch.Tensor, n_dim: int):
    """[B, S, K] / [B, S, N] -> contiguous-row 2-D views (KRN:1026-1032)."""
    if x.dim() != 3 or out.dim() != 3:
        raise ValueError(f"x and out must be [B, S, *]; got {tuple(x.shape)} and {tuple(out.shape)}")
    bsz, seqlen, m_dim = x.shape
    if tuple(out.shape[:2]) != (bsz, seqlen):
        raise ValueError(f"out {tuple(out.shape)} does not match x {tuple(x.shape)}")
    bt = bsz * seqlen
    x2d = x.reshape(bt, m_dim)
    if x2d.stride(-1) != 1 or x2d.stride(0) % 8 != 0 or x2d.data_ptr() % 16 != 0 or m_dim % 8 != 0:
        x2d = x2d.contiguous()
    if not out.is_contiguous():
        raise ValueError("out must be contiguous (results would otherwise be written to a temporary)")
    y2d = out.view(bt, n_dim)
    return x2d, y2d, bt, m_dim


def _pad_k(x2d: torch.Tensor) -> torch.Tensor:
    k = x2d.shape[1]
    if k % 8 == 0 and x2d.stride(0) % 8 == 0 and x2d.data_ptr() % 16 == 0:
        return x2d
    kp = (k + 7) // 8 * 8
    xp = torch.zeros((x2d.shape[0], kp), dtype=x2d.dtype, device=x2d.device)
    xp[:, :k] = x2d
    return xp


def _check_shapes(x2d: torch.Tensor, weight: torch.Tensor, y2d: torch.Tensor, n_dim: int, m_dim: int) -> None:
    if tuple(weight.shape) != (n_dim, m_dim):
        raise ValueError(f"weight must be [N={n_dim}, K={m_dim}] (nn.Linear layout), got {tuple(weight.shape)}")
    if not (x2d.dtype == weight.dtype == y2d.dtype):
        raise TypeError(f"dtype mismatch: x {x2d.dtype}, weight {weight.dtype}, out {y2d.dtype}")
    _dtype_code(x2d)


def gemm_packed(x2d: torch.Tensor, packed: torch.Tensor, n_dim: int, active_blocks: Optional[torch.Tensor],
                y2d: torch.Tensor, *, num_active: Optional[int] = None, num_active_dev: Optional[torch.Tensor] = None,
                bitmap: Optional[torch.Tensor] = None, total_k_blocks: Optional[int] = None,
                plan: Optional[Plan] = None, workspace_prefix: str = "gemm",
                kernel: Optional[_KernelHandle] = None, sort_list: bool = False) -> Plan:
    """Launch one block-sparse GEMM on already packed weights (2-D x [bt, K], y [bt, N]).

    Exactly one source of active blocks: `active_blocks` (int32 device list, host length or
    `num_active`; optional device count), `bitmap` (u8), or neither (dense: every block).
    sort_list: the GEMM sorts the list ascending itself (bsg_gemm_sorted, at most
    MAX_NBLK // 2 entries), with the result of an ascending sort followed by the GEMM.  With
    `num_active_dev` the device count is applied first: only the first min(count, num_active)
    entries are sorted and used (the GEMM on sort(list[:count]), not on the count smallest ids)."""
    lib = load()
    dev = _require_cuda(x2d, packed, y2d)
    code = _dtype_code(x2d)
    bt, k_dim = x2d.shape
    x2d = _pad_k(x2d)
    nblk = int(packed.shape[0])
    if (k_dim + BLOCK_K - 1) // BLOCK_K != nblk:
        raise ValueError(f"x has K={k_dim} but the packed weight has {nblk} K-blocks")
    if y2d.shape[0] != bt or y2d.shape[1] != n_dim or y2d.stride(1) != 1:
        raise ValueError("y must be [bt, N] with unit column stride")
    if bt == 0:
        return Plan()
    stream = _stream_handle(dev)
    if bitmap is not None:
        mode = "bitmap"
        nbm = int(total_k_blocks if total_k_blocks is not None else bitmap.numel())
        na_for_plan = nbm
    elif active_blocks is not None:
        mode = "list"
        na = int(active_blocks.numel() if num_active is None else num_active)
        if na > (MAX_NBLK // 2 if sort_list else MAX_NBLK):
            raise ValueError(f"{na} active blocks exceeds {MAX_NBLK // 2 if sort_list else MAX_NBLK}"
                             + (" (in-kernel sort)" if sort_list else ""))
        na_for_plan = na
    else:
        mode = "dense"
        na_for_plan = nblk
    if mode == "list":
        if active_blocks.dtype != torch.int32:
            active_blocks = active_blocks.to(torch.int32)
        active_blocks = active_blocks.contiguous()
    elif mode == "bitmap":
        if bitmap.dtype not in (torch.uint8, torch.bool, torch.int8):
            raise TypeError(f"bitmap must be uint8, got {bitmap.dtype}")
        bitmap = bitmap.contiguous()
        if bitmap.numel() < nbm or bitmap.device != dev:
            raise ValueError(f"bitmap must hold total_k_blocks={nbm} entries on {dev}")
    kd = x2d.shape[1]

    def launch(pl: Plan, ws_ptr, ws_bytes: int) -> int:
        with torch.cuda.device(dev):
            if mode == "list":
                nad = num_active_dev.data_ptr() if num_active_dev is not None else None
                entry = lib.bsg_gemm_sorted if sort_list else lib.bsg_gemm
                return entry(x2d.data_ptr(), x2d.stride(0), bt, kd, packed.data_ptr(), n_dim,
                                    active_blocks.data_ptr() if na > 0 else None, na, nad, y2d.data_ptr(),
                                    y2d.stride(0), code, ws_ptr, ws_bytes, ctypes_byref(pl), stream)
            if mode == "bitmap":
                return lib.bsg_gemm_bitmap(x2d.data_ptr(), x2d.stride(0), bt, kd, packed.data_ptr(), n_dim,
                                           bitmap.data_ptr(), nbm, y2d.data_ptr(), y2d.stride(0), code, ws_ptr,
                                           ws_bytes, ctypes_byref(pl), stream)
            return lib.bsg_gemm_dense(x2d.data_ptr(), x2d.stride(0), bt, kd, packed.data_ptr(), n_dim,
                                      y2d.data_ptr(), y2d.stride(0), code, ws_ptr, ws_bytes, ctypes_byref(pl), stream)

    pl = None
    if plan is None or not any(plan.as_tuple()):
        pl = _first_call_plan(bt, n_dim, nblk, na_for_plan, mode, code, dev, _tuning_launcher(lib, bt, n_dim, dev, launch))
    if pl is None:
        pl = resolve_plan(bt, n_dim, nblk, na_for_plan, dev, plan, dense=(mode == "dense"))
    ws_bytes = int(lib.bsg_gemm_workspace_bytes(bt, n_dim, ctypes_byref(pl)))
    ws_ptr = (_workspace(workspace_prefix, dev, ws_bytes, (bt, n_dim) + pl.as_tuple()).data_ptr()
              if ws_bytes > 0 else None)
    check(launch(pl, ws_ptr, ws_bytes))
    if kernel is not None:
        kernel.last_plan = pl
    return pl


def _tuning_launcher(lib, bt: int, n_dim: int, dev: torch.device, launch):
    """launch(plan) for first-call tuning: one scratch workspace (grown as candidates need, freed
    with the closure), its counters cleared whenever the candidate changes, since the previous
    candidate's partials may lie where this one's counters start."""
    state = {"buf": None, "last": None}

    def run(pl: Plan) -> int:
        need = int(lib.bsg_gemm_workspace_bytes(bt, n_dim, ctypes_byref(pl)))
        if need < 0:
            return need
        if need == 0:
            return launch(pl, None, 0)
        buf = state["buf"]
        if buf is None or buf.numel() < need:
            buf = state["buf"] = torch.zeros(need, dtype=torch.uint8, device=dev)
            state["last"] = pl.as_tuple()
        elif state["last"] != pl.as_tuple():
            rc = lib.bsg_workspace_init(buf.data_ptr(), buf.numel(), _stream_handle(dev))
            if rc != _lib.BSG_OK:
                return rc
            state["last"] = pl.as_tuple()
        return launch(pl, buf.data_ptr(), buf.numel())

    return run


def _first_call_plan(bt: int, n_dim: int, nblk: int, na: int, mode: str, code: int, dev: torch.device,
                     launch) -> Optional[Plan]:
    """For a problem the tuned table does not cover: the plan first-call tuning chose for its key
    (tuned now, on this call's buffers, unless a stream is being captured or tuning is off), or
    None (table plan or library heuristics)."""
    from . import autotune, tuning

    if tuning.lookup(bt, n_dim, nblk, na, dense=(mode == "dense")) is not None:
        return None
    k = autotune.key(n_dim, nblk, bt, na, mode, code)
    pl = autotune.cached(k)
    if pl is not None or not autotune.enabled() or torch.cuda.is_current_stream_capturing():
        return pl
    cands = tuning.candidate_plans(bt, na, nblk)
    heuristic = resolve_plan(bt, n_dim, nblk, na, dev, None, dense=(mode == "dense"), lookup_plan=False)
    if heuristic.as_tuple() not in {c.as_tuple() for c in cands}:
        cands.append(heuristic)
    return autotune.tune(k, cands, launch, dev)


def _sort_active_blocks_asc(active_blocks: torch.Tensor) -> torch.Tensor:
    """Ascending sort of the block list (KRN:140-163, GPU path)."""
    if int(active_blocks.numel()) <= 1:
        return active_blocks
    if active_blocks.dtype != torch.int32:
        active_blocks = active_blocks.to(torch.int32)
    return torch.sort(active_blocks.contiguous())[0].contiguous()


class _PreparedCall:
    """One eager call site of the drop-in, resolved once: the launch arguments that depend only on
    the problem (packed weight, plan, workspace, sizes), kept with references to the packed weight
    and the workspace so that neither is freed while the entry lives.  A hit re-checks only what
    the key does not pin (the weight's identity, storage and version; alignment and contiguity; the
    current device) and passes the call's own pointers and stream."""

    __slots__ = ("wref", "wptr", "wver", "fn", "wp", "ldx", "bt", "kd", "n", "na", "ldy", "code", "ws", "ws_bytes",
                 "plan", "plan_ref", "dev_index", "keep", "kernel")

    def launch(self, x: torch.Tensor, ab: torch.Tensor, out: torch.Tensor) -> None:
        rc = self.fn(x.data_ptr(), self.ldx, self.bt, self.kd, self.wp, self.n, ab.data_ptr(), self.na, None,
                     out.data_ptr(), self.ldy, self.code, self.ws, self.ws_bytes, self.plan_ref,
                     torch._C._cuda_getCurrentRawStream(self.dev_index))
        if rc != _lib.BSG_OK:
            check(rc)
        self.kernel.last_plan = self.plan


_PREPARED: Dict[tuple, _PreparedCall] = {}
_PREPARED_MAX = 4096


# Other prepared-call caches (the model patch's) register their clear here.
_FORGET_HOOKS: list = []


def forget_prepared_calls() -> None:
    """Drop every prepared call (their plans came from tuning state that is being reset, or hold
    packed weights that are being released)."""
    _PREPARED.clear()
    for hook in _FORGET_HOOKS:
        hook()


def _prepared_key(x, weight, active_blocks, out, cache_prefix, sort_active_blocks, active_blocks_limit) -> tuple:
    return (cache_prefix, id(weight), x.shape, x.stride(), x.dtype, x.get_device(), out.shape, out.dtype,
            out.get_device(), active_blocks.shape, active_blocks.dtype, active_blocks.get_device(),
            sort_active_blocks, active_blocks_limit)


def _prepare_call(key, x, weight, entry, active_blocks, out, x2d, y2d, num_blocks, sort_list, pl, ws_prefix) -> None:
    """Record the call just launched through the general path, when its form needs no per-call
    work: no copy of x, an int32 contiguous list passed as given (the caller excludes a list sorted
    by a torch.sort launch), not under capture (where first-call tuning is deferred)."""
    if (torch.cuda.is_current_stream_capturing() or x2d.data_ptr() != x.data_ptr() or not x.is_contiguous()
            or active_blocks.dtype != torch.int32 or not active_blocks.is_contiguous()):
        return
    lib = load()
    code = _dtype_code(x2d)
    ws_bytes = int(lib.bsg_gemm_workspace_bytes(x2d.shape[0], y2d.shape[1], ctypes_byref(pl)))
    ws = (_workspace(ws_prefix, x2d.device, ws_bytes, (x2d.shape[0], y2d.shape[1]) + pl.as_tuple())
          if ws_bytes > 0 else None)
    c = _PreparedCall()
    c.wref = entry.ref
    c.wptr = int(weight.data_ptr())
    c.wver = entry.version
    c.fn = lib.bsg_gemm_sorted if sort_list else lib.bsg_gemm
    c.wp = int(entry.packed.data_ptr())
    c.ldx, c.bt, c.kd = int(x2d.stride(0)), int(x2d.shape[0]), int(x2d.shape[1])
    c.n, c.na, c.ldy, c.code = int(y2d.shape[1]), int(num_blocks), int(y2d.stride(0)), code
    c.ws = ws.data_ptr() if ws is not None else None
    c.ws_bytes = ws_bytes
    c.plan = Plan(*pl.as_tuple())
    c.plan_ref = ctypes_byref(c.plan)
    c.dev_index = x2d.device.index if x2d.device.index is not None else torch.cuda.current_device()
    c.keep = (entry.packed, ws)
    c.kernel = prepacked_block_sparse_gemm_batched_kernel
    if len(_PREPARED) >= _PREPARED_MAX:
        _PREPARED.clear()
    _PREPARED[key] = c


def _prepacked_block_sparse_gemm_from_active_blocks(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_blocks: torch.Tensor,
    out: torch.Tensor,
    cache_prefix: str = "gemm",
    proj_tag: str = "",
    sort_active_blocks: bool = True,
    use_run_compressed: bool = True,
    active_blocks_limit: Optional[int] = None,
) -> None:
    """Y = X[:, active K-blocks] · W[active K-blocks, :] into `out` (KRN:3166-3344).

    `active_blocks_limit` keeps the first that many list entries (KRN:3179, 3191-3192);
    `use_run_compressed` and `proj_tag` only selected Triton metadata variants and are
    accepted for signature compatibility (the HIP kernel streams the list as given).

    A repeated call site (same weight, shapes, dtypes, devices and options) takes a prepared
    launch: the packed weight, plan and workspace resolved by its first call, with only the
    weight's identity and version, the alignment and contiguity of x, out and the list, and the
    current device re-checked before the one library call."""
    key = _prepared_key(x, weight, active_blocks, out, cache_prefix, sort_active_blocks, active_blocks_limit)
    pc = _PREPARED.get(key)
    if pc is not None:
        if (pc.wref() is weight and weight._version == pc.wver and weight.data_ptr() == pc.wptr
                and x.data_ptr() % 16 == 0 and out.is_contiguous() and active_blocks.is_contiguous()
                and torch._C._cuda_getDevice() == pc.dev_index):
            pc.launch(x, active_blocks, out)
            return
        del _PREPARED[key]
    n_dim = out.shape[-1]
    num_blocks = int(active_blocks.numel()) if active_blocks_limit is None else int(active_blocks_limit)
    num_blocks = min(num_blocks, int(active_blocks.numel()))
    if num_blocks <= 0:
        out.zero_()
        return
    x2d, y2d, bt, m_dim = _views(x, out, n_dim)
    _check_shapes(x2d, weight, y2d, n_dim, m_dim)
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    ab = active_blocks
    if ab.dtype != torch.int32:
        ab = ab.to(torch.int32)
    ab = ab.contiguous()
    # the GEMM reads the first num_blocks entries; it sorts them itself (no sort launch) up to
    # MAX_NBLK // 2 of them
    in_kernel = sort_active_blocks and num_blocks <= MAX_NBLK // 2
    if sort_active_blocks and not in_kernel:
        ab = _sort_active_blocks_asc(ab[:num_blocks])
    pl = gemm_packed(x2d, entry.packed, n_dim, ab, y2d, num_active=num_blocks, plan=None,
                     workspace_prefix=f"{cache_prefix}_ws", kernel=prepacked_block_sparse_gemm_batched_kernel,
                     sort_list=in_kernel)
    if ab is active_blocks and (in_kernel or not sort_active_blocks):
        _prepare_call(key, x, weight, entry, active_blocks, out, x2d, y2d, num_blocks, in_kernel, pl,
                      f"{cache_prefix}_ws")


def _prepacked_block_sparse_gemm_from_active_blocks_splitk(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_blocks: torch.Tensor,
    out: torch.Tensor,
    cache_prefix: str = "gemm_1d_sk",
    num_split_k: Optional[int] = None,
    tile_b: Optional[int] = None,
    tile_n: Optional[int] = None,
    tile_warps: Optional[int] = None,
    tile_stages: Optional[int] = None,
) -> None:
    """List-driven GEMM with an explicit split-K factor and tile (KRN:1350-1454)."""
    n_dim = out.shape[-1]
    if int(active_blocks.numel()) <= 0:
        out.zero_()
        return
    x2d, y2d, bt, m_dim = _views(x, out, n_dim)
    _check_shapes(x2d, weight, y2d, n_dim, m_dim)
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    plan = make_plan(num_split_k, tile_b, tile_n, tile_warps, tile_stages, bt=bt)
    gemm_packed(x2d, entry.packed, n_dim, active_blocks, y2d, plan=plan, workspace_prefix=f"{cache_prefix}_ws",
                kernel=prepacked_block_sparse_gemm_batched_kernel)


def _build_active_k_bitmap(active_blocks: torch.Tensor, total_k_blocks: int, device) -> torch.Tensor:
    """u8 bitmap with 1 at every active block (KRN:1056-1061)."""
    bitmap = torch.zeros(int(total_k_blocks), dtype=torch.uint8, device=device)
    if int(active_blocks.numel()) > 0:
        bitmap[active_blocks.to(torch.long)] = 1
    return bitmap


def _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_blocks: torch.Tensor,
    out: torch.Tensor,
    cache_prefix: str = "gemm_bpl",
    total_k_blocks: Optional[int] = None,
    prebuilt_bitmap: Optional[torch.Tensor] = None,
) -> None:
    """Bitmap-driven GEMM (KRN:1064-1147): the bitmap is compacted into an ascending block
    list inside the kernel, so blocks are summed in ascending order as in KRN:845-871."""
    _bitmap_gemm(x, weight, active_blocks, out, cache_prefix, total_k_blocks, prebuilt_bitmap, None,
                 prepacked_block_sparse_gemm_bitmap_preload_batched_kernel)


def _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk(
    x: torch.Tensor,
    weight: torch.Tensor,
    active_blocks: torch.Tensor,
    out: torch.Tensor,
    cache_prefix: str = "gemm_bpl_sk",
    total_k_blocks: Optional[int] = None,
    prebuilt_bitmap: Optional[torch.Tensor] = None,
    num_split_k: Optional[int] = None,
    tile_b: Optional[int] = None,
    tile_n: Optional[int] = None,
    tile_warps: Optional[int] = None,
    tile_stages: Optional[int] = None,
) -> None:
    """Bitmap-driven GEMM with an explicit split-K factor and tile (KRN:1235-1347)."""
    plan = make_plan(num_split_k, tile_b, tile_n, tile_warps, tile_stages, bt=int(x.shape[0]) * int(x.shape[1]))
    _bitmap_gemm(x, weight, active_blocks, out, cache_prefix, total_k_blocks, prebuilt_bitmap, plan,
                 prepacked_block_sparse_gemm_bitmap_preload_batched_kernel)


def _bitmap_gemm(x, weight, active_blocks, out, cache_prefix, total_k_blocks, prebuilt_bitmap, plan, kernel) -> None:
    n_dim = out.shape[-1]
    if int(active_blocks.numel()) <= 0:
        out.zero_()
        return
    x2d, y2d, bt, m_dim = _views(x, out, n_dim)
    _check_shapes(x2d, weight, y2d, n_dim, m_dim)
    if total_k_blocks is None:
        total_k_blocks = (m_dim + BLOCK_K - 1) // BLOCK_K
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    bitmap = prebuilt_bitmap if prebuilt_bitmap is not None else _build_active_k_bitmap(
        active_blocks, total_k_blocks, x.device)
    gemm_packed(x2d, entry.packed, n_dim, None, y2d, bitmap=bitmap, total_k_blocks=int(total_k_blocks), plan=plan,
                workspace_prefix=f"{cache_prefix}_ws", kernel=kernel)


def dense_gemm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, cache_prefix: str = "gemm_dense",
               plan: Optional[Plan] = None) -> None:
    """The same kernel with every K-block active: the in-run dense baseline."""
    n_dim = out.shape[-1]
    x2d, y2d, bt, m_dim = _views(x, out, n_dim)
    _check_shapes(x2d, weight, y2d, n_dim, m_dim)
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    gemm_packed(x2d, entry.packed, n_dim, None, y2d, plan=plan, workspace_prefix=f"{cache_prefix}_ws")


# ---------------------------------------------------------------------------------------
# Tile enumeration (the reference's autotune config list, KRN:636-674)


def kernel_tiles() -> Sequence[tuple]:
    """Instantiated (kind, rows_per_group, cols_per_wave, waves_per_group, depth) tuples."""
    out = []
    for kind in (1, 2, 3, 4, 5, 6, 7):
        for rows in ((1, 2, 4, 8) if kind == 3 else (16, 32, 64)):
            for cols in ((16, 32, 48, 64, 96) if kind >= 5 else (16, 32, 64, 128)):
                for waves in (1, 2, 4, 8):
                    for depth in (1, 2, 4, 8):
                        p = Plan(1, cols, waves, depth, rows, kind)
                        if load().bsg_plan_resolve(rows, cols, 1, 1, 1, ctypes_byref(p)) == _lib.BSG_OK:
                            out.append((kind, rows, cols, waves, depth))
    return out


def __getattr__(name: str):
    if name == "_PREPACK_AUTOTUNE_CONFIGS":
        cfgs = [TileConfig({"BLOCK_B": r, "BLOCK_N": Plan(1, c, w, d, r, k).group_cols()}, num_warps=w,
                           num_stages=d, kind=k) for (k, r, c, w, d) in kernel_tiles()]
        globals()[name] = cfgs
        return cfgs
    raise AttributeError(name)


def n_keep_for_density(density: float, total_k: int) -> int:
    """Number of kept blocks for a density (scripts/bench_roundrobin_e2e_decode.py:102)."""
    return max(1, min(int(total_k), int(round(float(density) * int(total_k)))))


def active_bytes(na: int, n: int, dtype_bytes: int = 2) -> int:
    """Algorithmic active-weight bytes of one GEMM: na * 64 * N * dtype_bytes."""
    return int(na) * BLOCK_K * int(n) * int(dtype_bytes)


def nblk_of(k: int) -> int:
    return int(math.ceil(int(k) / BLOCK_K))
