"""First-call autotuning for problems the shipped plan table does not cover.

The reference's GEMM kernels are Triton-autotuned on the key (N_OUT, M, BATCHSIZE,
NUM_ACTIVE_BLOCKS) (kernels/shared_mask_batched_triton_min_runtime.py:684-687, configs
KRN:636-674): the first call with a new key times every config on that call's own arguments and
later calls reuse the winner, which `kernel.best_config` reports (scripts/profile_kernel_configs.py:135).
This module does the same for a GEMM whose shape has no entry in `tuned_plans.json`: every
instantiated plan for the batch's row bucket (`tuning.candidate_plans`) is launched on the call's
own buffers, the fastest few are timed again, and the winner is kept per key (problem shape,
block count, batch, active blocks, block source, dtype).  The key's plan can be persisted to a
JSON file (`set_autotune(cache_path=...)` or BSA_MI355X_AUTOTUNE_CACHE) and is loaded from it.

Tuning launches only on the current stream and synchronizes, so it never runs while a stream is
being captured: a capture with an untuned key uses the library's heuristics.  BSA_MI355X_AUTOTUNE=0
turns first-call tuning off (table plan, else heuristics, as before).
"""
from __future__ import annotations

import json
import os
import statistics
import threading
from typing import Callable, Dict, List, Optional, Tuple

import torch

from ._lib import BSG_OK, Plan

Key = Tuple[int, int, int, int, str, int]

_STATE = {
    "enabled": os.environ.get("BSA_MI355X_AUTOTUNE", "1") != "0",
    "path": os.environ.get("BSA_MI355X_AUTOTUNE_CACHE") or None,
    "loaded": False,
    "tunes": 0,
    "timed_launches": 0,
}
_CACHE: Dict[Key, Tuple[Plan, float]] = {}
_LOCK = threading.Lock()


def key(n: int, nblk: int, bt: int, na: int, mode: str, dtype_code: int) -> Key:
    """The tuning key: output columns, K-blocks, batch rows, active blocks (the block count for
    dense), block source ('list', 'bitmap', 'dense') and dtype."""
    return (int(n), int(nblk), int(bt), int(na), str(mode), int(dtype_code))


def enabled() -> bool:
    return bool(_STATE["enabled"])


def set_autotune(enabled: bool = True, cache_path: Optional[str] = None) -> None:
    """Turn first-call tuning on or off; with cache_path, load tuned keys from that JSON file
    (when it exists) and write every new one back to it."""
    from .runtime import forget_prepared_calls

    with _LOCK:
        _STATE["enabled"] = bool(enabled)
        if cache_path is not None:
            _STATE["path"] = cache_path
            _STATE["loaded"] = False
    _load()
    forget_prepared_calls()


def stats() -> dict:
    """Keys tuned in this process and candidate launches timed for them."""
    return {"keys": len(_CACHE), "tunes": _STATE["tunes"], "timed_launches": _STATE["timed_launches"]}


def clear() -> None:
    from .runtime import forget_prepared_calls

    with _LOCK:
        _CACHE.clear()
        _STATE["tunes"] = 0
        _STATE["timed_launches"] = 0
    forget_prepared_calls()


def cached(k: Key) -> Optional[Plan]:
    _load()
    hit = _CACHE.get(k)
    return None if hit is None else Plan(*hit[0].as_tuple())


def record(k: Key, plan: Plan, us: float) -> None:
    with _LOCK:
        _CACHE[k] = (Plan(*plan.as_tuple()), float(us))
    _save()


def _load() -> None:
    path = _STATE["path"]
    if _STATE["loaded"] or not path:
        return
    with _LOCK:
        _STATE["loaded"] = True
        if not os.path.exists(path):
            return
        with open(path) as f:
            data = json.load(f)
        for e in data.get("entries", []):
            k = tuple(e["key"])
            if len(k) != 6:
                continue
            _CACHE.setdefault((int(k[0]), int(k[1]), int(k[2]), int(k[3]), str(k[4]), int(k[5])),
                              (Plan(*[int(v) for v in e["plan"]]), float(e.get("us", 0.0))))


def _save() -> None:
    path = _STATE["path"]
    if not path:
        return
    with _LOCK:
        entries = [{"key": list(k), "plan": list(p.as_tuple()), "us": round(us, 3)} for k, (p, us) in
                   sorted(_CACHE.items())]
        tmp = f"{path}.tmp{os.getpid()}"
        with open(tmp, "w") as f:
            json.dump({"entries": entries}, f, indent=1)
        os.replace(tmp, path)


def tune(k: Key, candidates: List[Plan], launch: Callable[[Plan], int], device: torch.device,
         reps: int = 3, finalists: int = 4, final_reps: int = 10) -> Optional[Plan]:
    """Time every candidate with `launch(plan) -> status` on the current stream (one warm-up
    launch, then `reps` back to back between two events), re-time the `finalists` fastest with
    `final_reps` launches each, record and return the fastest.  Candidates the library rejects
    (non-zero status on the warm-up launch) are skipped; None when none runs."""
    stream = torch.cuda.current_stream(device)

    def timed(p: Plan, n: int) -> float:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            launch(p)
        b.record(stream)
        b.synchronize()
        _STATE["timed_launches"] += n
        return a.elapsed_time(b) * 1000.0 / n

    first = []
    for p in candidates:
        if launch(p) != BSG_OK:
            continue
        first.append((timed(p, reps), p))
    if not first:
        return None
    first.sort(key=lambda t: t[0])
    fin = [p for _, p in first[:finalists]]
    samples = {i: [] for i in range(len(fin))}
    for _ in range(3):
        for i, p in enumerate(fin):
            samples[i].append(timed(p, final_reps))
    i = min(samples, key=lambda j: statistics.median(samples[j]))
    best, us = fin[i], statistics.median(samples[i])
    _STATE["tunes"] += 1
    record(k, best, us)
    return Plan(*best.as_tuple())
