"""Model integration: route a Llama-style model's decode-time linears through the sparse GEMM.

Reference counterpart: scripts/bench_roundrobin_e2e_decode.py (RRD) -- `_sparse_linear`
(RRD:179-284), `_patch_roundrobin_sparse` (RRD:287-503), `_restore` (RRD:506-508) and their
helpers `_nearest_cfg` (RRD:74-79), `_get_module` (RRD:82-86), PROJS / PROJ_TO_SHAPE
(RRD:39-48).  The same names, arguments, return values and statistics keys live here; a driver
switches by importing them.  Behaviour kept from the reference:

  * a call with more than one token per sequence (prefill), or a density >= 1, runs the
    module's dense `F.linear` (the dense-prefill bypass);
  * a decode call selects blocks with the reference's rules (`_select_active_blocks`) and runs
    the GEMM on them.  By default both are one library call (bsg_select_gemm_rule: the score
    launch, then a GEMM whose work-groups rank the scores themselves), with the plan of the
    lookup-table entry (its split-K and tile; naive and bpl sum the kept blocks in the same
    ascending order here).  With profile_sparse_parts (the reference times selection and GEMM
    apart) or fixed masks, selection and GEMM run as separate calls, the GEMM through the kernel
    family the entry names (naive / bpl, split-K, tile), as in RRD:207-276;
  * the optional energy gate (modes dense / expand / scaled / hybrid), mask reuse, per-step
    density schedules and weight-aware scores behave as there.

Every device step is this package's HIP code (selector kernels, GEMM kernels); only the
control flow around them is Python, as in the reference.
"""
from __future__ import annotations

import time
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from .runtime import (_FORGET_HOOKS, INDEX_BLOCK_META_SIZE, _build_active_k_bitmap, _check_shapes, _get_prepacked_weight_block_major,
                      _packed_entry, _prepacked_block_sparse_gemm_from_active_blocks,
                      _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload,
                      _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk,
                      _prepacked_block_sparse_gemm_from_active_blocks_splitk, _views, make_plan,
                      n_keep_for_density)
from .select import (_energy_expanded_active_blocks, _prior_or_none, _select_active_blocks, _topk_energy_ratio,
                     prepare_select_gemm_rule)

PROJS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]
PROJ_TO_SHAPE = {"q_proj": "qkvo", "k_proj": "qkvo", "v_proj": "qkvo", "o_proj": "qkvo",
                 "gate_proj": "gate_up", "up_proj": "gate_up", "down_proj": "down"}


def _nearest_cfg(sweep: dict, shape: str, density: float) -> dict:
    """The lookup-table row of `shape` whose density key is nearest to `density`, copied, with
    the key recorded under "density_key" (RRD:74-79)."""
    rows = sweep[shape]
    key = min(rows, key=lambda k: abs(float(k) - float(density)))
    cfg = dict(rows[key])
    cfg["density_key"] = key
    return cfg


def _get_module(model, layer_idx: int, proj: str):
    """model.model.layers[i].self_attn.<q/k/v/o>_proj or .mlp.<gate/up/down>_proj (RRD:82-86)."""
    layer = model.model.layers[layer_idx]
    return getattr(layer.self_attn if proj in PROJS[:4] else layer.mlp, proj)


def _as_decode3(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(x.shape[0], 1, x.shape[-1]) if x.dim() == 2 else x


def _sync_time(enabled: bool) -> Optional[float]:
    if not enabled:
        return None
    torch.cuda.synchronize()
    return time.perf_counter()


def _sparse_linear(x, weight, density: float, cfg: dict, cache_prefix: str, block_k: int, stats: dict,
                   profile_sparse_parts: bool, bitmap_buf: Optional[torch.Tensor],
                   block_prior: Optional[torch.Tensor] = None, prior_alpha: float = 1.0, prior_eps: float = 0.1,
                   fixed_active_blocks: Optional[torch.Tensor] = None,
                   block_score_scale: Optional[torch.Tensor] = None):
    """y = x · Wᵀ over the selected K-blocks for a decode call; dense `F.linear` for prefill
    (more than one token per sequence) or density >= 1 (RRD:179-284).  `cfg` is a lookup-table
    row: best_kern "naive" (block list) or "bpl" (bitmap), best_K (split-K), best_tile."""
    x3 = _as_decode3(x)
    if x3.shape[1] != 1 or density >= 1.0:
        return F.linear(x, weight)
    n_out, d_in = int(weight.shape[0]), int(weight.shape[1])
    total_k = d_in // block_k
    if fixed_active_blocks is None and not profile_sparse_parts:
        out = torch.empty(x3.shape[0], x3.shape[1], n_out, device=x3.device, dtype=x3.dtype)
        _fused_select_linear(x3, weight, out, density, cfg, cache_prefix, block_k, block_prior, prior_alpha,
                             prior_eps, block_score_scale)
        stats["calls"] += 1
        return out.reshape(x.shape[0], n_out) if x.dim() == 2 else out

    t0 = _sync_time(profile_sparse_parts)
    if fixed_active_blocks is not None:
        active = fixed_active_blocks.to(device=x3.device, dtype=torch.int32)
    else:
        active = _select_active_blocks(x3, density, block_k, block_prior, prior_alpha, prior_eps, block_score_scale)
    if t0 is not None:
        stats["select_wall_s"] = stats.get("select_wall_s", 0.0) + (_sync_time(True) - t0)

    out = torch.empty(x3.shape[0], x3.shape[1], n_out, device=x3.device, dtype=x3.dtype)
    kern = str(cfg["best_kern"])
    split_k = int(cfg.get("best_K") or 1)
    tb, tn, nw, ns = cfg.get("best_tile") or [None, None, None, None]
    t1 = _sync_time(profile_sparse_parts)
    if kern == "naive":
        if split_k <= 1:
            _prepacked_block_sparse_gemm_from_active_blocks(x3, weight, active, out, cache_prefix=cache_prefix,
                                                            use_run_compressed=False)
        else:
            _prepacked_block_sparse_gemm_from_active_blocks_splitk(
                x3, weight, active, out, cache_prefix=cache_prefix, num_split_k=split_k, tile_b=tb, tile_n=tn,
                tile_warps=nw, tile_stages=ns)
    else:
        if bitmap_buf is not None and int(bitmap_buf.numel()) == total_k:
            bitmap = bitmap_buf
            bitmap.zero_()
            if int(active.numel()) > 0:
                bitmap[active.to(torch.long)] = 1
        else:
            bitmap = _build_active_k_bitmap(active, total_k, x3.device)
        if split_k <= 1:
            _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload(
                x3, weight, active, out, cache_prefix=cache_prefix, total_k_blocks=total_k, prebuilt_bitmap=bitmap)
        else:
            _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk(
                x3, weight, active, out, cache_prefix=cache_prefix, total_k_blocks=total_k, prebuilt_bitmap=bitmap,
                num_split_k=split_k, tile_b=tb, tile_n=tn, tile_warps=nw, tile_stages=ns)
    stats["calls"] += 1
    if t1 is not None:
        dt = _sync_time(True) - t1
        stats["wall_s"] += dt
        stats["kernel_wall_s"] = stats.get("kernel_wall_s", 0.0) + dt
    return out.reshape(x.shape[0], n_out) if x.dim() == 2 else out


class _PreparedLinear:
    """One decode call site of `_fused_select_linear` resolved once (packed weight, options with
    device copies of the prior and scale, plan, workspace: select.RuleCall).  A hit re-checks
    what its key does not pin: the weight's identity, storage and version, the prior's and the
    scale's versions, x's alignment and the current device."""

    __slots__ = ("call", "wref", "wptr", "wver", "prior", "prior_ver", "scale", "scale_ver", "dev_index")

    def valid(self, x3, weight, block_prior, block_score_scale) -> bool:
        return (self.wref() is weight and weight._version == self.wver and weight.data_ptr() == self.wptr
                and block_prior is self.prior and (block_prior is None or block_prior._version == self.prior_ver)
                and block_score_scale is self.scale
                and (block_score_scale is None or block_score_scale._version == self.scale_ver)
                and x3.data_ptr() % 16 == 0 and torch._C._cuda_getDevice() == self.dev_index)


_PREPARED_LINEAR: Dict[tuple, _PreparedLinear] = {}
_FORGET_HOOKS.append(_PREPARED_LINEAR.clear)


def _fused_select_linear(x3, weight, out, density: float, cfg: dict, cache_prefix: str, block_k: int,
                         block_prior, prior_alpha: float, prior_eps: float, block_score_scale) -> None:
    """The reference's selection (`_select_active_blocks`, RRD:90-113: mean L2 norm, or the
    channel-scaled energy with block_score_scale; the prior when it has floor(K/64) entries;
    n_keep = max(1, min(nblk, round(density * nblk)))) and the GEMM on the kept blocks, as one
    library call on the packed weight of `cache_prefix` (the select -> bitmap -> GEMM of
    RRD:207-276 without the host-side steps between them).  The lookup row's split-K and tile
    become the plan; a naive row without split-K takes the tuned table's plan.  A repeated call
    site (same weight, x shape, density, lookup row, prior and scale) reuses its resolved call."""
    key = (cache_prefix, id(weight), x3.shape, x3.stride(), x3.dtype, x3.get_device(), float(density),
           str(cfg.get("best_kern")), cfg.get("best_K"), tuple(cfg.get("best_tile") or ()), id(block_prior),
           id(block_score_scale), float(prior_alpha), float(prior_eps), int(block_k))
    pc = _PREPARED_LINEAR.get(key)
    if pc is not None and out.is_contiguous():
        if pc.valid(x3, weight, block_prior, block_score_scale):
            pc.call.launch(x3.data_ptr(), out.data_ptr(), torch._C._cuda_getCurrentRawStream(pc.dev_index))
            return
        del _PREPARED_LINEAR[key]
    if int(block_k) != INDEX_BLOCK_META_SIZE:
        raise ValueError(f"block_k must be {INDEX_BLOCK_META_SIZE}")
    n_out = out.shape[-1]
    x2d, y2d, bt, d_in = _views(x3, out, n_out)
    _check_shapes(x2d, weight, y2d, n_out, d_in)
    split_k = int(cfg.get("best_K") or 1)
    tb, tn, nw, ns = cfg.get("best_tile") or [None, None, None, None]
    plan = None
    if str(cfg["best_kern"]) != "naive" or split_k > 1:
        plan = make_plan(split_k if split_k > 1 else None, tb, tn, nw, ns, bt=bt)
        if not any(plan.as_tuple()):
            plan = None
    entry = _packed_entry(weight, block_k, cache_prefix)
    call = prepare_select_gemm_rule(x2d, entry.packed, n_out, n_keep_for_density(density, d_in // block_k), y2d,
                                    score="energy" if block_score_scale is not None else "l2_mean",
                                    block_prior=_prior_or_none(block_prior, x2d), prior_alpha=prior_alpha,
                                    prior_eps=prior_eps, channel_scale=block_score_scale, plan=plan,
                                    workspace_prefix=f"{cache_prefix}_selrule_ws")
    dev = x2d.device
    with torch.cuda.device(dev):
        call.launch(x2d.data_ptr(), y2d.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    if x2d.data_ptr() == x3.data_ptr() and x3.is_contiguous() and not torch.cuda.is_current_stream_capturing():
        pc = _PreparedLinear()
        pc.call = call
        pc.wref = entry.ref
        pc.wptr = int(weight.data_ptr())
        pc.wver = entry.version
        pc.prior, pc.scale = block_prior, block_score_scale
        pc.prior_ver = block_prior._version if block_prior is not None else 0
        pc.scale_ver = block_score_scale._version if block_score_scale is not None else 0
        pc.dev_index = dev.index if dev.index is not None else torch.cuda.current_device()
        if len(_PREPARED_LINEAR) >= 4096:
            _PREPARED_LINEAR.clear()
        _PREPARED_LINEAR[key] = pc


class _SparseForward:
    """The replacement forward of one (layer, projection) linear: decode calls go through
    `_sparse_linear` with this cell's density, lookup row, prior and gate (RRD:331-499)."""

    def __init__(self, owner: "_PatchState", mod, layer: int, proj: str, density: float, schedule,
                 block_score_scale, bitmap_buf, orig):
        self.owner, self.mod, self.layer, self.proj = owner, mod, layer, proj
        self.density, self.schedule = float(density), schedule
        self.block_score_scale, self.bitmap_buf, self.orig = block_score_scale, bitmap_buf, orig
        self.key = (layer, proj)
        self.cfg = _nearest_cfg(owner.sweep, PROJ_TO_SHAPE[proj], self.density)

    def _prefix(self, cfg: dict) -> str:
        return f"rr_e2e_l{self.layer}_{self.proj}_{cfg['best_kern']}"

    def _run(self, x, density: float, cfg: dict, prior, fixed=None):
        o = self.owner
        return _sparse_linear(x, self.mod.weight, density, cfg, self._prefix(cfg), o.block_k, o.stats,
                              o.profile_sparse_parts, self.bitmap_buf, prior, o.prior_alpha, o.prior_eps, fixed,
                              self.block_score_scale)

    def _step_density(self, x) -> Tuple[float, dict]:
        """Per-step schedule: decode call c uses schedule[1 + c mod (len - 1)] (entry 0 belongs
        to the dense prefill), so repeated timing runs replay the same schedule."""
        if self.schedule is None or _as_decode3(x).shape[1] != 1:
            return self.density, self.cfg
        calls = self.owner.decode_call_counts.get(self.key, 0)
        self.owner.decode_call_counts[self.key] = calls + 1
        n = len(self.schedule)
        i = (calls % (n - 1)) + 1 if n > 1 else 0
        d = float(self.schedule[i] if i < n else self.schedule[-1])
        return d, _nearest_cfg(self.owner.sweep, PROJ_TO_SHAPE[self.proj], d)

    def _gate_keep(self) -> Optional[float]:
        o = self.owner
        if o.energy_gate_keep_by_cell is not None and self.key in o.energy_gate_keep_by_cell:
            return float(o.energy_gate_keep_by_cell[self.key])
        return None if o.energy_gate_keep is None else float(o.energy_gate_keep)

    def _cell_stat(self, density: float) -> dict:
        return self.owner.cell_energy_stats.setdefault(f"{self.layer}:{self.proj}", {
            "layer": int(self.layer), "proj": str(self.proj), "density": float(density), "checks": 0,
            "ratio_sum": 0.0, "ratio_min": 1.0, "ratio_max": 0.0, "dense_fallbacks": 0, "expands": 0,
            "scaled_fallbacks": 0})

    def _gated(self, x, density: float, keep: float, prior):
        """The energy gate (RRD:360-455): when the top-k blocks hold less than `keep` of the
        batch-mean energy, expand the list, scale the sparsity down, or run dense.  Returns
        None when the gate passes."""
        o, st = self.owner, self.owner.stats
        ratio = _topk_energy_ratio(x, density, o.block_k, prior, o.prior_alpha, o.prior_eps)
        st["energy_gate_checks"] = st.get("energy_gate_checks", 0) + 1
        st["energy_gate_ratio_sum"] = st.get("energy_gate_ratio_sum", 0.0) + float(ratio)
        cell = self._cell_stat(density)
        cell["checks"] += 1
        cell["ratio_sum"] += float(ratio)
        cell["ratio_min"] = min(float(cell["ratio_min"]), float(ratio))
        cell["ratio_max"] = max(float(cell["ratio_max"]), float(ratio))
        if ratio >= keep:
            return None
        mode = o.energy_gate_mode
        if mode == "expand" or (mode == "hybrid" and o.energy_gate_expand_projs is not None
                                and self.proj in o.energy_gate_expand_projs):
            active, exp_ratio, exp_density = _energy_expanded_active_blocks(
                x, density, o.block_k, keep, prior, o.prior_alpha, o.prior_eps)
            st["energy_gate_expands"] = st.get("energy_gate_expands", 0) + 1
            st["energy_gate_expanded_ratio_sum"] = st.get("energy_gate_expanded_ratio_sum", 0.0) + float(exp_ratio)
            st["energy_gate_expanded_density_sum"] = (st.get("energy_gate_expanded_density_sum", 0.0)
                                                      + float(exp_density))
            cell["expands"] += 1
            cfg2 = _nearest_cfg(o.sweep, PROJ_TO_SHAPE[self.proj], float(exp_density))
            return self._run(x, float(exp_density), cfg2, None, fixed=active)
        if mode == "scaled":
            base = min(1.0, max(0.0, 1.0 - density))
            fallback_s = min(1.0, max(0.0, min(base, base * float(o.energy_gate_fallback_sparsity_scale))))
            d2 = max(density, min(1.0, 1.0 - fallback_s))
            st["energy_gate_scaled_fallbacks"] = st.get("energy_gate_scaled_fallbacks", 0) + 1
            st["energy_gate_scaled_density_sum"] = st.get("energy_gate_scaled_density_sum", 0.0) + float(d2)
            cell["scaled_fallbacks"] += 1
            return self._run(x, float(d2), _nearest_cfg(o.sweep, PROJ_TO_SHAPE[self.proj], float(d2)), prior)
        st["energy_gate_dense_fallbacks"] = st.get("energy_gate_dense_fallbacks", 0) + 1
        cell["dense_fallbacks"] += 1
        return self.orig(x)

    def __call__(self, x):
        o = self.owner
        prior = o.block_priors.get(self.key)
        density, cfg = self._step_density(x)
        cached = o.reuse_masks and self.key in o.mask_cache
        keep = self._gate_keep()
        if keep is not None and density < 1.0 and not cached:
            gated = self._gated(x, density, keep, prior)
            if gated is not None:
                return gated
        if cached:
            return self._run(x, density, cfg, None, fixed=o.mask_cache[self.key])
        out = self._run(x, density, cfg, prior)
        if o.reuse_masks and density < 1.0 and self.key not in o.mask_cache:
            x3 = _as_decode3(x)
            if x3.shape[1] == 1:
                o.mask_cache[self.key] = _select_active_blocks(x3, density, o.block_k, prior, o.prior_alpha,
                                                               o.prior_eps, self.block_score_scale)
        return out


class _PatchState:
    """Settings and mutable state shared by every patched linear of one model."""

    def __init__(self, sweep, profile_sparse_parts, block_priors, prior_alpha, prior_eps, reuse_masks,
                 energy_gate_keep, energy_gate_keep_by_cell, energy_gate_mode, energy_gate_expand_projs,
                 energy_gate_fallback_sparsity_scale):
        self.sweep = sweep
        self.profile_sparse_parts = bool(profile_sparse_parts)
        self.block_priors = block_priors or {}
        self.prior_alpha, self.prior_eps = float(prior_alpha), float(prior_eps)
        self.reuse_masks = bool(reuse_masks)
        self.energy_gate_keep = energy_gate_keep
        self.energy_gate_keep_by_cell = energy_gate_keep_by_cell
        self.energy_gate_mode = energy_gate_mode
        self.energy_gate_expand_projs = energy_gate_expand_projs
        self.energy_gate_fallback_sparsity_scale = energy_gate_fallback_sparsity_scale
        self.block_k = max(16, int(INDEX_BLOCK_META_SIZE))
        self.cell_energy_stats: Dict[str, dict] = {}
        self.stats = {"calls": 0, "wall_s": 0.0, "cell_energy_stats": self.cell_energy_stats}
        self.mask_cache: Dict[tuple, torch.Tensor] = {}
        self.decode_call_counts: Dict[tuple, int] = {}


def _patch_roundrobin_sparse(model, alloc, sweep, profile_sparse_parts: bool,
                             block_priors: Optional[dict] = None, prior_alpha: float = 1.0, prior_eps: float = 0.1,
                             reuse_masks: bool = False, energy_gate_keep: Optional[float] = None,
                             energy_gate_keep_by_cell: Optional[Dict[tuple, float]] = None,
                             energy_gate_mode: str = "dense", energy_gate_expand_projs: Optional[set] = None,
                             energy_gate_fallback_sparsity_scale: float = 0.5, weight_aware_score: bool = False,
                             step_density_alloc: Optional[Dict[tuple, List[float]]] = None):
    """Replace the forward of every q/k/v/o/gate/up/down linear of `model` (RRD:287-503).
    `alloc[str(layer)][proj]` is the cell's density, `sweep[shape][density]` the lookup rows.
    Weights are packed up front for the prefixes the cell can use.  Returns (originals, stats)
    for `_restore` and for the caller's accounting."""
    state = _PatchState(sweep, profile_sparse_parts, block_priors, prior_alpha, prior_eps, reuse_masks,
                        energy_gate_keep, energy_gate_keep_by_cell, energy_gate_mode, energy_gate_expand_projs,
                        energy_gate_fallback_sparsity_scale)
    originals = []
    for li in range(len(model.model.layers)):
        for proj in PROJS:
            mod = _get_module(model, li, proj)
            density = float(alloc[str(li)][proj])
            schedule = (step_density_alloc or {}).get((li, proj))
            scale = None
            if weight_aware_score and density < 1.0:
                scale = mod.weight.detach().float().pow(2).sum(dim=0)  # per input channel
            fwd = _SparseForward(state, mod, li, proj, density, schedule, scale, None, mod.forward)
            kerns = {fwd.cfg["best_kern"]} | ({"naive", "bpl"} if schedule is not None else set())
            for kern in sorted(kerns):
                _get_prepacked_weight_block_major(mod.weight, state.block_k, cache_prefix=f"rr_e2e_l{li}_{proj}_{kern}")
            if (str(fwd.cfg["best_kern"]) == "bpl" and density < 1.0) or schedule is not None:
                fwd.bitmap_buf = torch.empty(int(mod.weight.shape[1]) // state.block_k, dtype=torch.uint8,
                                             device=mod.weight.device)
            originals.append((mod, mod.forward))
            mod.forward = fwd
    return originals, state.stats


def _restore(originals) -> None:
    """Put back the forwards `_patch_roundrobin_sparse` replaced (RRD:506-508)."""
    for mod, orig in originals:
        mod.forward = orig
