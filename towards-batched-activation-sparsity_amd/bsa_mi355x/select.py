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


_SCORES = {"l1": _lib.BSG_SCORE_L1, "l2_mean": _lib.BSG_SCORE_L2_MEAN, "energy": _lib.BSG_SCORE_ENERGY}


def _dev_f32(t: Optional[torch.Tensor], dev: torch.device, n: int, what: str, exact: bool = False) -> Optional[torch.Tensor]:
    if t is None:
        return None
    t = t.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if t.numel() < n or (exact and t.numel() != n):
        raise ValueError(f"{what} has {t.numel()} entries, needs {n}")
    return t


def _prior_or_none(block_prior: Optional[torch.Tensor], x: torch.Tensor) -> Optional[torch.Tensor]:
    """The reference applies a block prior only when it holds exactly floor(K/64) entries and
    silently ignores it otherwise (RRD:110-112, 135-138, 161-164)."""
    if block_prior is None or int(block_prior.numel()) != int(x.shape[-1]) // BLOCK_K:
        return None
    return block_prior


def _capacity(score: str, k: int, kd: int, energy_keep: float) -> int:
    """Entries the kept list may hold: every scored block (floor(K/64)) under an energy budget,
    else min(k, blocks) (ceil(K/64) blocks for the L1 rule, floor(K/64) for the reference's)."""
    nb = kd // BLOCK_K
    if score == "l1":
        return max(0, min(int(k), (kd + BLOCK_K - 1) // BLOCK_K))
    return nb if energy_keep > 0 else max(0, min(int(k), nb))


def _rule_opts(dev, kd: int, score: str, block_prior, prior_alpha: float, prior_eps: float, channel_scale,
               energy_keep: float, ratio_out: Optional[torch.Tensor]):
    """bsg_select_opts for a call, the ratio output (made when an energy budget is set and none
    was given) and the device tensors the options point at (kept alive by the caller)."""
    if score not in _SCORES:
        raise ValueError(f"score must be one of {sorted(_SCORES)}")
    want_ratio = ratio_out is not None or (score != "l1" and energy_keep > 0)
    if want_ratio and ratio_out is None:
        ratio_out = torch.empty(1, dtype=torch.float32, device=dev)
    prior = _dev_f32(block_prior, dev, kd // BLOCK_K, "block_prior", exact=True)
    # the reference reads block_score_scale[:d_eff] (RRD:104): one entry per scored channel
    scale = _dev_f32(channel_scale, dev, (kd // BLOCK_K) * BLOCK_K, "channel_scale")
    opts = _lib.SelectOpts(_SCORES[score], float(energy_keep), prior.data_ptr() if prior is not None else None,
                           float(prior_alpha), float(prior_eps), scale.data_ptr() if scale is not None else None,
                           ratio_out.data_ptr() if want_ratio else None)
    return opts, ratio_out, (prior, scale)


def select_topk(x: torch.Tensor, k: int, score: str = "l2_mean", block_prior: Optional[torch.Tensor] = None,
                prior_alpha: float = 1.0, prior_eps: float = 0.1, channel_scale: Optional[torch.Tensor] = None,
                energy_keep: float = 0.0, idx_out: Optional[torch.Tensor] = None,
                count_out: Optional[torch.Tensor] = None, ratio_out: Optional[torch.Tensor] = None,
                workspace_prefix: str = "select") -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Device selector with the reference's scoring rules (RRD:90-176), fp64 scores, ranking by
    (score desc, block id asc).  x is [..., K] fp16/bf16; blocks are floor(K/64).

    score "l2_mean" | "energy" | "l1"; block_prior multiplies the score by
    max(prior + eps, 1e-6)^alpha; channel_scale ([K]) weights the energy score; energy_keep > 0
    keeps the first ranks whose cumulative energy reaches that fraction (at least k).
    Returns (idx int32 ascending, padded to the capacity; count int32 [1]; ratio float32 [1] or
    None), all on the device: idx[:count] is the selection."""
    lib = load()
    dev = _require_cuda(x)
    x2d = _x2d(x)
    bt, kd = x2d.shape
    nb = kd // BLOCK_K
    if nb < 1:
        raise ValueError(f"K={kd} has no whole 64-channel block")
    if score not in _SCORES:
        raise ValueError(f"score must be one of {sorted(_SCORES)}")
    cap = _capacity(score, k, kd, energy_keep)
    if idx_out is None:
        idx_out = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    if count_out is None:
        count_out = torch.empty(1, dtype=torch.int32, device=dev)
    opts, ratio_out, _keep = _rule_opts(dev, kd, score, block_prior, prior_alpha, prior_eps, channel_scale,
                                        energy_keep, ratio_out)
    want_ratio = ratio_out is not None
    ws_bytes = int(lib.bsg_select_workspace_bytes(kd))
    ws = _workspace(workspace_prefix, dev, ws_bytes)
    with torch.cuda.device(dev):
        check(lib.bsg_select_topk(x2d.data_ptr(), x2d.stride(0), bt, kd, int(k), ctypes_byref(opts),
                                  idx_out.data_ptr(), count_out.data_ptr(), _dtype_code(x2d), ws.data_ptr(), ws_bytes,
                                  _stream_handle(dev)))
    return idx_out, count_out, (ratio_out if want_ratio else None)


def _select_active_blocks(x3: torch.Tensor, density: float, block_k: int = BLOCK_K,
                          block_prior: Optional[torch.Tensor] = None, prior_alpha: float = 1.0, prior_eps: float = 0.1,
                          block_score_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Drop-in for `_select_active_blocks` (scripts/bench_roundrobin_e2e_decode.py:90-113): the
    reference's score (mean L2 norm, or the channel-scaled energy when block_score_scale is
    given; optional prior), n_keep = max(1, min(nblk, round(density * nblk))), ascending int32
    ids on the device, one kernel launch."""
    if int(block_k) != BLOCK_K:
        raise ValueError(f"block_k must be {BLOCK_K}")
    nb = x3.shape[-1] // BLOCK_K
    nk = n_keep_for_density(density, nb)
    idx, _, _ = select_topk(x3, nk, score="energy" if block_score_scale is not None else "l2_mean",
                            block_prior=_prior_or_none(block_prior, x3), prior_alpha=prior_alpha, prior_eps=prior_eps,
                            channel_scale=block_score_scale, workspace_prefix="select_ref")
    return idx[:nk]


def _topk_energy_ratio(x: torch.Tensor, density: float, block_k: int = BLOCK_K,
                       block_prior: Optional[torch.Tensor] = None, prior_alpha: float = 1.0,
                       prior_eps: float = 0.1) -> float:
    """Drop-in for `_topk_energy_ratio` (RRD:116-141): the fraction of the batch-mean block
    energy kept by the top-n_keep blocks (energy score, optional prior).  Synchronises to
    return a float, as the reference does."""
    x3 = x.reshape(x.shape[0], 1, x.shape[-1]) if x.dim() == 2 else x
    if x3.shape[1] != 1 or density >= 1.0:
        return 1.0
    if int(block_k) != BLOCK_K:
        raise ValueError(f"block_k must be {BLOCK_K}")
    nb = x3.shape[-1] // BLOCK_K
    nk = n_keep_for_density(density, nb)
    ratio = torch.empty(1, dtype=torch.float32, device=x3.device)
    select_topk(x3, nk, score="energy", block_prior=_prior_or_none(block_prior, x3), prior_alpha=prior_alpha,
                prior_eps=prior_eps, ratio_out=ratio, workspace_prefix="select_ref")
    return float(ratio.item())


def _energy_expanded_active_blocks(x: torch.Tensor, density: float, block_k: int, energy_keep: float,
                                   block_prior: Optional[torch.Tensor] = None, prior_alpha: float = 1.0,
                                   prior_eps: float = 0.1):
    """Drop-in for `_energy_expanded_active_blocks` (RRD:144-176): top-n_keep blocks by energy
    (optional prior), grown to the first rank whose cumulative energy reaches energy_keep of
    the total.  Returns (ascending int32 ids, kept energy ratio, kept density) like the
    reference, which synchronises for the count."""
    x3 = x.reshape(x.shape[0], 1, x.shape[-1]) if x.dim() == 2 else x
    if x3.shape[1] != 1 or density >= 1.0:
        return None, 1.0, 1.0
    if int(block_k) != BLOCK_K:
        raise ValueError(f"block_k must be {BLOCK_K}")
    nb = x3.shape[-1] // BLOCK_K
    nk = n_keep_for_density(density, nb)
    idx, cnt, ratio = select_topk(x3, nk, score="energy", block_prior=_prior_or_none(block_prior, x3),
                                  prior_alpha=prior_alpha,
                                  prior_eps=prior_eps, energy_keep=float(energy_keep), workspace_prefix="select_ref")
    keep = int(cnt.item())
    return idx[:keep], float(ratio.item()), float(keep / nb)


def select_sparse_gemm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, k: int, cache_prefix: str = "sel_gemm",
                       plan=None, idx_out: Optional[torch.Tensor] = None,
                       count_out: Optional[torch.Tensor] = None, score: str = "l1", **rule) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused online selection + block-sparse GEMM: out = X[:, top-k blocks] · W[top-k blocks].

    x [B, S, K], weight nn.Linear [N, K], out [B, S, N].  score "l1" is the exact-L1 rule
    (select_gemm_packed); "l2_mean" or "energy" the reference's rules (select_gemm_rule_packed,
    which takes the options of `rule`: block_prior, prior_alpha, prior_eps, channel_scale,
    energy_keep, ratio_out).  One to three launches on the current stream, no host round trip;
    returns the (device) selected list and count."""
    n_dim = out.shape[-1]
    x2d, y2d, bt, m_dim = _views(x, out, n_dim)
    _check_shapes(x2d, weight, y2d, n_dim, m_dim)
    entry = _packed_entry(weight, BLOCK_K, cache_prefix)
    if score == "l1" and not rule:
        return select_gemm_packed(x2d, entry.packed, n_dim, k, y2d, plan=plan, idx_out=idx_out, count_out=count_out,
                                  workspace_prefix=f"{cache_prefix}_ws")
    idx, cnt, _ = select_gemm_rule_packed(x2d, entry.packed, n_dim, k, y2d, score=score, plan=plan, idx_out=idx_out,
                                          count_out=count_out, workspace_prefix=f"{cache_prefix}_ws", **rule)
    return idx, cnt


class RuleCall:
    """A select_gemm_rule_packed call resolved once: the bsg_select_opts with device copies of the
    prior and the channel scale, the plan, the workspace and the id / count / ratio outputs, kept
    alive with the object; launch(x_ptr, y_ptr, stream) then makes the one library call.  Valid
    for x of the same shape and strides (row stride ldx), the same packed weight, and prior and
    scale of unchanged values."""

    __slots__ = ("fn", "bt", "kd", "ldx", "k", "n", "ldy", "code", "wp", "opts", "opts_ref", "plan", "plan_ref",
                 "ws", "ws_bytes", "idx", "cnt", "ratio", "keep")

    def launch(self, x_ptr: int, y_ptr: int, stream: int) -> None:
        rc = self.fn(x_ptr, self.ldx, self.bt, self.kd, self.k, self.opts_ref, self.wp, self.n, self.idx.data_ptr(),
                     self.cnt.data_ptr(), y_ptr, self.ldy, self.code, self.ws, self.ws_bytes, self.plan_ref, stream)
        if rc != _lib.BSG_OK:
            check(rc)


def prepare_select_gemm_rule(x2d: torch.Tensor, packed: torch.Tensor, n_dim: int, k: int, y2d: torch.Tensor,
                             score: str = "l2_mean", block_prior: Optional[torch.Tensor] = None,
                             prior_alpha: float = 1.0, prior_eps: float = 0.1,
                             channel_scale: Optional[torch.Tensor] = None, energy_keep: float = 0.0, plan=None,
                             idx_out: Optional[torch.Tensor] = None, count_out: Optional[torch.Tensor] = None,
                             ratio_out: Optional[torch.Tensor] = None,
                             workspace_prefix: str = "sel_rule_ws") -> RuleCall:
    """Checks and resolves a select_gemm_rule_packed call (see there) without launching it."""
    lib = load()
    dev = _require_cuda(x2d, packed, y2d)
    bt, m_dim = x2d.shape
    if m_dim % 8 != 0 or x2d.stride(1) != 1 or x2d.stride(0) % 8 != 0:
        raise ValueError(f"x must be [bt, K] with unit column stride and K % 8 == 0 (K={m_dim})")
    nblk = int(packed.shape[0])
    if (m_dim + BLOCK_K - 1) // BLOCK_K != nblk:
        raise ValueError(f"x has K={m_dim} but the packed weight has {nblk} K-blocks")
    if m_dim // BLOCK_K < 1:
        raise ValueError(f"K={m_dim} has no whole 64-channel block")
    cap = _capacity(score, k, m_dim, energy_keep)
    if idx_out is None:
        idx_out = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    if count_out is None:
        count_out = torch.empty(1, dtype=torch.int32, device=dev)
    if int(idx_out.numel()) < cap:
        raise ValueError(f"idx_out holds {idx_out.numel()} ids, the selection may keep {cap}")
    opts, ratio_out, keep = _rule_opts(dev, m_dim, score, block_prior, prior_alpha, prior_eps, channel_scale,
                                       energy_keep, ratio_out)
    pl = resolve_plan(bt, n_dim, nblk, cap, dev, plan, select=True)
    sel_bytes = int(lib.bsg_select_workspace_bytes(m_dim))
    gemm_bytes = int(lib.bsg_gemm_workspace_bytes(bt, n_dim, ctypes_byref(pl)))
    ws = _workspace(workspace_prefix, dev, sel_bytes + gemm_bytes, (bt, n_dim) + pl.as_tuple())
    c = RuleCall()
    c.fn = lib.bsg_select_gemm_rule
    c.bt, c.kd, c.ldx, c.k = int(bt), int(m_dim), int(x2d.stride(0)), int(k)
    c.n, c.ldy, c.code, c.wp = int(n_dim), int(y2d.stride(0)), _dtype_code(x2d), int(packed.data_ptr())
    c.opts = opts
    c.opts_ref = ctypes_byref(opts)
    c.plan = pl
    c.plan_ref = ctypes_byref(pl)
    c.ws, c.ws_bytes = ws.data_ptr(), sel_bytes + gemm_bytes
    c.idx, c.cnt, c.ratio = idx_out, count_out, ratio_out
    c.keep = (keep, ws, packed)
    return c


def select_gemm_rule_packed(x2d: torch.Tensor, packed: torch.Tensor, n_dim: int, k: int, y2d: torch.Tensor,
                            score: str = "l2_mean", block_prior: Optional[torch.Tensor] = None,
                            prior_alpha: float = 1.0, prior_eps: float = 0.1,
                            channel_scale: Optional[torch.Tensor] = None, energy_keep: float = 0.0, plan=None,
                            idx_out: Optional[torch.Tensor] = None, count_out: Optional[torch.Tensor] = None,
                            ratio_out: Optional[torch.Tensor] = None, workspace_prefix: str = "sel_rule_ws"
                            ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Selection by the reference's rules (select_topk's options, RRD:90-176) + the GEMM on the
    kept blocks, one library call (bsg_select_gemm_rule): the kept ids, count and ratio are those
    select_topk gives for the same x and options, all on the device.  Two launches when the GEMM
    ranks the fp64 score keys itself (no energy budget, no ratio, fp16), else three.  Returns
    (idx int32 with room for the capacity, count [1], ratio [1] or None)."""
    c = prepare_select_gemm_rule(x2d, packed, n_dim, k, y2d, score, block_prior, prior_alpha, prior_eps,
                                 channel_scale, energy_keep, plan, idx_out, count_out, ratio_out, workspace_prefix)
    dev = x2d.device
    with torch.cuda.device(dev):
        c.launch(x2d.data_ptr(), y2d.data_ptr(), _stream_handle(dev))
    return c.idx, c.cnt, c.ratio


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
    pl = resolve_plan(bt, n_dim, nblk, kk, dev, plan, select=True)
    sel_bytes = int(lib.bsg_select_workspace_bytes(m_dim))
    gemm_bytes = int(lib.bsg_gemm_workspace_bytes(bt, n_dim, ctypes_byref(pl)))
    ws = _workspace(workspace_prefix, dev, sel_bytes + gemm_bytes, (bt, n_dim) + pl.as_tuple())
    with torch.cuda.device(dev):
        check(lib.bsg_select_gemm(x2d.data_ptr(), x2d.stride(0), bt, m_dim, int(k), packed.data_ptr(), n_dim,
                                  idx_out.data_ptr(), count_out.data_ptr(), y2d.data_ptr(), y2d.stride(0),
                                  _dtype_code(x2d), ws.data_ptr(), sel_bytes + gemm_bytes, ctypes_byref(pl),
                                  _stream_handle(dev)))
    return idx_out[:kk], count_out
