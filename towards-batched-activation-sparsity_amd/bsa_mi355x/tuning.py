"""Launch-plan tuning: profile plans on the GPU, ship the best per shape, look them up at run time.

Counterpart of the reference's config search and lookup tables:
  * scripts/profile_kernel_configs.py:86-216 searches (kernel, split-K, tile) per batch size,
    shape and density and writes llama2_kernel_best_sweep_B{bs}.json
    ({shape: {density: {mask, block_k, K, tile, dense_ms, sparse_ms, speedup}}}, :293-296);
  * scripts/bench_perstep_actual_kernel_speedup.py:90-112 and
    scripts/bench_roundrobin_e2e_decode.py:75-80, 218-221 read those tables, the latter with
    the other key set (best_kern, best_K, best_tile).
Here the search runs over this library's plans (kind, rows, columns, waves, depth, split-K),
each timed as a hipGraph of back-to-back launches rotating over >= 1 GiB of packed-weight copies
(so the 256 MB Infinity Cache cannot serve repeats).  `tune()` writes
  * a flat table (tuned_plans.json, shipped next to this file) used by `lookup()`, which
    `runtime.resolve_plan` consults whenever the caller gives no plan, and
  * optionally per-batch files in the reference's lookup layout carrying BOTH key sets, so the
    reference's drivers can consume them; `load_reference_lookup()` reads either key set back.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import time
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

from ._lib import BLOCK_K, Plan

TABLE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuned_plans.json")

LLAMA2_7B_SHAPES = {"qkvo": (4096, 4096), "gate_up": (4096, 11008), "down": (11008, 4096),
                    # q/k/v and gate/up fused along N (one GEMM per shared input and mask)
                    "qkv_fused": (4096, 12288), "gate_up_fused": (4096, 22016)}

_TABLE: Optional[List[dict]] = None
_INDEX: Dict[Tuple[int, int], List[dict]] = {}
# lookup() answers per (bt, N, nblk, na, dense, select), cleared whenever a table is loaded
_MEMO: Dict[tuple, Optional[tuple]] = {}


def rows_bucket(bt: int) -> int:
    return 16 if bt <= 16 else (32 if bt <= 32 else 64)


# ---------------------------------------------------------------------------------------
# Run-time lookup


def load_table(path: str = TABLE_PATH) -> List[dict]:
    """Load a flat plan table ({"entries": [{bt, N, K, na, plan, us}, ...]}); missing -> []."""
    global _TABLE, _INDEX
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        data = {"entries": []}
    entries = [e for e in data.get("entries", []) if len(e.get("plan", ())) == 6]
    _TABLE = entries
    _INDEX = {}
    _MEMO.clear()
    from .runtime import forget_prepared_calls

    forget_prepared_calls()
    for e in entries:
        _INDEX.setdefault((int(e["N"]), (int(e["K"]) + BLOCK_K - 1) // BLOCK_K), []).append(e)
    return entries


def lookup(bt: int, n: int, nblk: int, na: int, dense: bool = False, select: bool = False) -> Optional[Plan]:
    """Best tabulated plan for (bt, N, nblk, na): same N and block count, same 16/32/64-row
    bucket, nearest batch, then the dense entry (dense=True) or the nearest active-block count.
    select=True (a selection + GEMM, whose GEMM ranks the block scores itself) prefers the
    entries timed that way (refine_select) and falls back to the plain GEMM's.  None when the
    shape is not tabulated."""
    if _TABLE is None:
        load_table()
    key = (int(bt), int(n), int(nblk), int(na), bool(dense), bool(select))
    if key in _MEMO:
        hit = _MEMO[key]
        return None if hit is None else Plan(*hit)
    p = _lookup(*key)
    _MEMO[key] = None if p is None else p.as_tuple()
    return p


def _lookup(bt: int, n: int, nblk: int, na: int, dense: bool, select: bool) -> Optional[Plan]:
    cands = _INDEX.get((n, nblk))
    if not cands:
        return None
    rb = rows_bucket(bt)
    same = [e for e in cands if rows_bucket(int(e["bt"])) == rb]
    if select and not dense:
        sel = [e for e in same if e.get("select")]
        if sel:
            same = sel
        else:
            same = [e for e in same if not e.get("select")]
    else:
        same = [e for e in same if not e.get("select")]
    if not same:
        return None
    best_bt = min({int(e["bt"]) for e in same}, key=lambda b: (abs(b - bt), b))
    same = [e for e in same if int(e["bt"]) == best_bt and bool(e.get("dense", False)) == bool(dense)]
    if not same:
        return None
    e = min(same, key=lambda e: (abs(int(e["na"]) - na), int(e["na"])))
    p = Plan(*[int(v) for v in e["plan"]])
    # a plan may split the batch into row groups only as it was tuned: groups of half the
    # bucket's rows (16 in the 32-row bucket, 32 in the 64-row one); never smaller tiles
    if p.rows_per_group < min(bt, 64) and not (rb >= 32 and p.rows_per_group == rb // 2):
        return None
    return p


# ---------------------------------------------------------------------------------------
# Reference lookup tables (both key sets)


def plan_from_reference_cfg(cfg: dict, bt: int) -> Optional[Plan]:
    """Plan for one reference lookup entry; None for "dense" entries.

    Accepts {mask, K, tile} (scripts/profile_kernel_configs.py:137-147) and {best_kern, best_K,
    best_tile} (scripts/bench_roundrobin_e2e_decode.py:218-221); an entry written by tune()
    also carries this library's own "plan", which wins."""
    from .runtime import make_plan

    if "plan" in cfg and len(cfg["plan"]) == 6:
        return Plan(*[int(v) for v in cfg["plan"]])
    mask = str(cfg.get("mask", cfg.get("best_kern", "")))
    if mask == "dense":
        return None
    split_k = int(cfg.get("K", cfg.get("best_K", 1)) or 1)
    tile = cfg.get("tile", cfg.get("best_tile")) or [None, None, None, None]
    tb, tn, nw, ns = (list(tile) + [None] * 4)[:4]
    return make_plan(split_k, tb, tn, nw, ns, bt=bt)


def load_reference_lookup(path: str) -> Dict[str, Dict[float, dict]]:
    """Read a llama2_kernel_best_sweep_B{bs}.json in either key set: {shape: {density: cfg}}
    with float density keys and every entry normalised to carry mask/K/tile."""
    with open(path) as f:
        data = json.load(f)
    out: Dict[str, Dict[float, dict]] = {}
    for shape, rows in data.items():
        if not isinstance(rows, dict):
            continue
        norm = {}
        for key, cfg in rows.items():
            try:
                d = float(key)
            except ValueError:
                continue
            c = dict(cfg)
            c.setdefault("mask", c.get("best_kern"))
            c.setdefault("K", c.get("best_K", 1))
            c.setdefault("tile", c.get("best_tile"))
            norm[d] = c
        out[shape] = norm
    return out


def nearest_density_cfg(table: Dict[float, dict], density: float) -> Tuple[float, dict]:
    """Nearest profiled density entry (scripts/bench_perstep_actual_kernel_speedup.py:56-57)."""
    key = min(table.keys(), key=lambda k: abs(float(k) - float(density)))
    return key, table[key]


# ---------------------------------------------------------------------------------------
# Profiling (GPU)


def candidate_plans(bt: int, na: int, nblk: int) -> List[Plan]:
    """Every instantiated tile for the batch bucket x split-K factors that leave >= 1 block per
    list splitter, plus the dot-product tiles (kind 3, no split-K) for batches of up to 8 rows."""
    from .runtime import kernel_tiles

    rb = rows_bucket(bt)
    fma_rows = 1 << max(0, (int(bt) - 1).bit_length()) if bt <= 8 else 0
    out = []
    for kind, rows, cols, waves, depth in kernel_tiles():
        if kind == 3:
            if rows == fma_rows:
                out.append(Plan(1, cols, waves, depth, rows, kind))
            continue
        if kind >= 5:  # variable-width column groups: the chip is filled without split-K
            # 32- and 64-row batches also try two row groups of half the rows (as below)
            if rows == rb or (rb >= 32 and rows == rb // 2):
                out.append(Plan(1, cols, waves, depth, rows, kind))
            continue
        # 32-row batches also try 64-row tiles; 32- and 64-row batches also try two row groups of
        # half the rows, which read each weight block twice, concurrently, but fill the chip
        # without split-K
        if rows != rb and not (rb == 32 and rows == 64) and not (rb >= 32 and rows == rb // 2):
            continue
        for sk in (1, 2, 3, 4, 6, 8):
            if sk * (waves if kind == 1 else 1) > max(na, 1):
                continue
            out.append(Plan(sk, cols, waves, depth, rows, kind))
    return out


def _rotation(active_bytes: int, rotate_bytes: int) -> int:
    """Launches per timing graph so that one replay reads >= rotate_bytes of distinct active weight."""
    return max(1, math.ceil(rotate_bytes / max(1, int(active_bytes))))


class _Case:
    """One (shape, batch) under tuning: packed-weight copies for the smallest active-block count
    that will be timed (min_na), inputs, and a block list set per density."""

    def __init__(self, bt: int, k: int, n: int, na: int, seed: int, device, rotate_bytes: int, min_na: int = 0):
        import torch

        from .runtime import pack_weight

        g = torch.Generator(device="cpu").manual_seed(seed)
        self.bt, self.k, self.n, self.na = bt, k, n, na
        self.nblk = (k + BLOCK_K - 1) // BLOCK_K
        self.rotate_bytes = rotate_bytes
        w = (torch.randn(k, n, generator=g) * 0.02).to(torch.float16).to(device)
        p0 = pack_weight(w, layout="kn")
        del w
        copies = _rotation(max(1, min_na or na) * BLOCK_K * n * 2, rotate_bytes)
        self.packed = [p0] + [p0.clone() for _ in range(copies - 1)]
        self.x = torch.randn(bt, k, generator=g).to(torch.float16).to(device)
        perm = torch.randperm(self.nblk, generator=g)[: max(na, 0)]
        self.idx = perm.sort()[0].to(torch.int32).to(device)
        self.y = torch.empty(bt, n, dtype=torch.float16, device=device)

    def time(self, plan: Optional[Plan], dense: bool = False, reps: int = 5, select: bool = False) -> float:
        """Median µs per launch over `reps` graph replays of R rotated launches, R copies holding
        >= rotate_bytes of the blocks this launch reads (so the Infinity Cache serves no repeat).
        select=True times the exact-L1 selection (k = the case's block count) + GEMM instead."""
        import torch

        from .runtime import gemm_packed
        from .select import select_gemm_packed

        na = self.nblk if dense else int(self.idx.numel())
        use = self.packed[: min(len(self.packed), _rotation(na * BLOCK_K * self.n * 2, self.rotate_bytes))]
        if select:
            sel_idx = torch.empty(max(na, 1), dtype=torch.int32, device=self.x.device)
            sel_cnt = torch.empty(1, dtype=torch.int32, device=self.x.device)

        def run():
            for p in use:
                if select:
                    select_gemm_packed(self.x, p, self.n, na, self.y, plan=plan, idx_out=sel_idx, count_out=sel_cnt,
                                       workspace_prefix="tune_sel")
                else:
                    gemm_packed(self.x, p, self.n, None if dense else self.idx, self.y, plan=plan,
                                workspace_prefix="tune")

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            run()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run()
        graph.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b) * 1000.0 / len(use))
        del graph
        return statistics.median(ts)


def _time_or_inf(case: "_Case", plan: Plan, dense: bool = False, select: bool = False) -> float:
    """A candidate the library rejects for this case (BsgUnsupported) never wins."""
    from ._lib import BsgUnsupported

    try:
        return case.time(plan, dense=dense, select=select)
    except BsgUnsupported:
        return float("inf")


def _pick(case: "_Case", plans: Sequence[Plan], dense: bool = False, margin: float = 0.05, finalists: int = 4,
          rounds: int = 3, select: bool = False) -> Tuple[float, Optional[Plan]]:
    """Best plan for a case: every candidate is timed once; those within `margin` of the best
    (at most `finalists`) are timed `rounds` more times, interleaved, and the lowest median wins
    (one timing each lets plans a few percent apart swap places from run to run)."""
    first = sorted(((us, p) for p in plans for us in [_time_or_inf(case, p, dense=dense, select=select)]
                    if math.isfinite(us)), key=lambda t: t[0])
    if not first:
        return float("inf"), None
    fin = [t for t in first if t[0] <= first[0][0] * (1.0 + margin)][:finalists]
    if len(fin) == 1:
        return fin[0]
    samples = [[us] for us, _ in fin]
    for _ in range(rounds):
        for i, (_, p) in enumerate(fin):
            samples[i].append(case.time(p, dense=dense, select=select))
    i = min(range(len(fin)), key=lambda j: statistics.median(samples[j]))
    return statistics.median(samples[i]), fin[i][1]


def tune(shapes: Dict[str, Tuple[int, int]], batch_sizes: Sequence[int], densities: Sequence[float],
         out_table: str = TABLE_PATH, lookup_dir: Optional[str] = None, rotate_bytes: int = 1 << 30,
         seed: int = 1234, log=print, merge_from: Optional[str] = None) -> List[dict]:
    """Profile every candidate plan for shape x batch x density; write the flat table (and the
    per-batch reference-layout lookups when lookup_dir is given).  Active blocks per density:
    max(1, floor(density * nblk)) as in scripts/profile_kernel_configs.py:111."""
    import torch

    dev = torch.device("cuda", torch.cuda.current_device())
    entries: List[dict] = []
    lookups: Dict[int, dict] = {}
    t_start = time.time()
    for sname, (k, n) in shapes.items():
        nblk = (k + BLOCK_K - 1) // BLOCK_K
        for bt in batch_sizes:
            min_na = min(max(1, min(nblk, int(math.floor(float(d) * nblk)))) for d in densities) if densities else nblk
            case = _Case(bt, k, n, nblk, seed, dev, rotate_bytes, min_na=min_na)
            dense_best = _pick(case, candidate_plans(bt, nblk, nblk), dense=True)
            entries.append({"shape": sname, "bt": bt, "N": n, "K": k, "na": nblk, "dense": True,
                            "plan": list(dense_best[1].as_tuple()), "us": round(dense_best[0], 3)})
            gen = torch.Generator().manual_seed(seed)
            for d in densities:
                na = max(1, min(nblk, int(math.floor(float(d) * nblk))))
                case.idx = torch.randperm(nblk, generator=gen)[:na].sort()[0].to(torch.int32).to(dev)
                best = _pick(case, candidate_plans(bt, na, nblk))
                entries.append({"shape": sname, "bt": bt, "N": n, "K": k, "na": na, "dense": False,
                                "plan": list(best[1].as_tuple()), "us": round(best[0], 3)})
                t = best[1]
                tile = [t.rows_per_group, t.group_cols(), t.waves_per_group, t.depth]
                rec = {"mask": "naive", "block_k": BLOCK_K, "K": t.split_k, "tile": tile,
                       "best_kern": "naive", "best_K": t.split_k, "best_tile": tile,
                       "dense_ms": dense_best[0] / 1000.0, "sparse_ms": best[0] / 1000.0,
                       "speedup": dense_best[0] / best[0], "plan": list(t.as_tuple()), "active_blocks": na}
                lookups.setdefault(bt, {}).setdefault(sname, {})[f"{float(d):.1f}"] = rec
                log(f"[tune {time.time() - t_start:6.1f}s] {sname} B={bt} d={d:.1f} na={na}: {best[0]:.2f} us "
                    f"plan={t.as_tuple()} (dense {dense_best[0]:.2f} us)")
            del case
            torch.cuda.empty_cache()
    meta = {"device": torch.cuda.get_device_name(dev), "rotate_bytes": rotate_bytes, "seed": seed}
    if merge_from:
        # keep the other (shape, batch) entries of an existing table
        tuned = {(e["shape"], e["bt"]) for e in entries}
        with open(merge_from) as f:
            old = json.load(f)
        entries = [e for e in old.get("entries", []) if (e["shape"], e["bt"]) not in tuned] + entries
    with open(out_table, "w") as f:
        json.dump({"meta": meta, "entries": entries}, f, indent=1)
    if lookup_dir:
        os.makedirs(lookup_dir, exist_ok=True)
        for bt, data in lookups.items():
            with open(os.path.join(lookup_dir, f"llama2_kernel_best_sweep_B{bt}.json"), "w") as f:
                json.dump(data, f, indent=1)
    load_table(out_table)
    return entries


def refine(shapes: Sequence[str], batch_sizes: Sequence[int], kinds: Sequence[int] = (5, 6),
           table: str = TABLE_PATH, out_table: Optional[str] = None, rotate_bytes: int = 1 << 30, seed: int = 1234,
           margin: float = 0.03, log=print) -> List[dict]:
    """Re-time the shipped table's entries for the given shapes and batches against the candidate
    plans of `kinds` (the kernels added after the table was made), keeping a new plan only when it
    beats the shipped one by more than `margin` on the same case (both timed in one run)."""
    import torch

    dev = torch.device("cuda", torch.cuda.current_device())
    with open(table) as f:
        data = json.load(f)
    entries = data["entries"]
    t_start = time.time()
    for sname in shapes:
        k, n = LLAMA2_7B_SHAPES[sname]
        nblk = (k + BLOCK_K - 1) // BLOCK_K
        for bt in batch_sizes:
            rows = [e for e in entries if e["shape"] == sname and int(e["bt"]) == bt and not e.get("select")]
            if not rows:
                continue
            min_na = min(int(e["na"]) for e in rows)
            case = _Case(bt, k, n, nblk, seed, dev, rotate_bytes, min_na=min_na)
            gen = torch.Generator().manual_seed(seed)
            for e in sorted(rows, key=lambda e: (not e["dense"], int(e["na"]))):
                na = int(e["na"])
                dense = bool(e["dense"])
                case.idx = torch.randperm(nblk, generator=gen)[:na].sort()[0].to(torch.int32).to(dev)
                old = Plan(*e["plan"])
                cands = [p for p in candidate_plans(bt, na, nblk) if p.kind in kinds]
                best_us, best = _pick(case, [old] + cands, dense=dense)
                old_us = statistics.median([case.time(old, dense=dense) for _ in range(3)])
                new_us = statistics.median([case.time(best, dense=dense) for _ in range(3)]) if best else float("inf")
                if best is not None and best.as_tuple() != old.as_tuple() and new_us < old_us * (1.0 - margin):
                    e["plan"], e["us"] = list(best.as_tuple()), round(new_us, 3)
                    verdict = "replaced"
                else:
                    e["us"] = round(old_us, 3)
                    verdict = "kept"
                log(f"[refine {time.time() - t_start:6.1f}s] {sname} B={bt} na={na}{' dense' if dense else ''}: "
                    f"{verdict} {old.as_tuple()} {old_us:.2f} us vs {best.as_tuple() if best else None} {new_us:.2f} us")
            del case
            torch.cuda.empty_cache()
    with open(out_table or table, "w") as f:
        json.dump(data, f, indent=1)
    load_table(out_table or table)
    return entries


def refine_select(shapes: Sequence[str], batch_sizes: Sequence[int], table: str = TABLE_PATH,
                  out_table: Optional[str] = None, rotate_bytes: int = 1 << 30, seed: int = 1234,
                  shortlist: int = 12, log=print) -> List[dict]:
    """Add or re-time the selection + GEMM entries ("select": true) of the table: for every sparse
    entry of the given shapes and batches, the exact-L1 selection of that many blocks followed by
    the GEMM that ranks the scores itself (select.select_gemm_packed, rotated like the GEMM's
    entries) is timed with the `shortlist` plans that are fastest as a plain GEMM and the plain
    GEMM's tabulated plan, and the fastest is kept.  The in-GEMM rank costs a work-group a cold load of the scores plus nblk^2
    compares spread over its waves, so the best plan can differ from the plain GEMM's."""
    import torch

    dev = torch.device("cuda", torch.cuda.current_device())
    with open(table) as f:
        data = json.load(f)
    entries = data["entries"]
    t_start = time.time()
    for sname in shapes:
        k, n = LLAMA2_7B_SHAPES[sname]
        nblk = (k + BLOCK_K - 1) // BLOCK_K
        for bt in batch_sizes:
            rows = [e for e in entries if e["shape"] == sname and int(e["bt"]) == bt and not e["dense"]
                    and not e.get("select")]
            if not rows:
                continue
            min_na = min(int(e["na"]) for e in rows)
            case = _Case(bt, k, n, nblk, seed, dev, rotate_bytes, min_na=min_na)
            gen = torch.Generator().manual_seed(seed)
            for e in sorted(rows, key=lambda e: int(e["na"])):
                na = int(e["na"])
                case.idx = torch.randperm(nblk, generator=gen)[:na].sort()[0].to(torch.int32).to(dev)
                base = Plan(*e["plan"])
                # every candidate timed as a plain GEMM first; the `shortlist` fastest (and the plain
                # GEMM's tabulated plan) are then timed as selection + GEMM
                plain = sorted(((us, p) for p in candidate_plans(bt, na, nblk) for us in [_time_or_inf(case, p)]
                                if math.isfinite(us)), key=lambda t: t[0])
                cands = [base] + [p for _, p in plain[:shortlist] if p.as_tuple() != base.as_tuple()]
                best_us, best = _pick(case, cands, select=True)
                base_us = statistics.median([case.time(base, select=True) for _ in range(3)])
                old = [x for x in entries if x.get("select") and x["shape"] == sname and int(x["bt"]) == bt
                       and int(x["na"]) == na]
                for x in old:
                    entries.remove(x)
                plan = best if best is not None else base
                entries.append({"shape": sname, "bt": bt, "N": n, "K": k, "na": na, "dense": False, "select": True,
                                "plan": list(plan.as_tuple()), "us": round(best_us if best else base_us, 3)})
                log(f"[select {time.time() - t_start:6.1f}s] {sname} B={bt} na={na}: {plan.as_tuple()} "
                    f"{best_us:.2f} us (plain GEMM's plan {base.as_tuple()}: {base_us:.2f} us)")
            del case
            torch.cuda.empty_cache()
    with open(out_table or table, "w") as f:
        json.dump(data, f, indent=1)
    load_table(out_table or table)
    return entries


def main(argv: Optional[Iterable[str]] = None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shapes", default="qkvo,gate_up,down")
    ap.add_argument("--batch-sizes", default="2,16,64")
    ap.add_argument("--densities", default="0.1,0.2,0.3,0.4,0.5,0.6,0.7,0.8,0.9")
    ap.add_argument("--out", default=TABLE_PATH)
    ap.add_argument("--lookup-dir", default=None)
    ap.add_argument("--merge", action="store_true",
                    help="keep the other (shape, batch) entries of the shipped table in the output")
    ap.add_argument("--refine-kinds", default=None,
                    help="instead of a full search, re-time the shipped entries against these kinds (e.g. 5,6)")
    ap.add_argument("--table", default=TABLE_PATH, help="--refine-kinds / --select: the table to start from")
    ap.add_argument("--select", action="store_true",
                    help="add the selection + GEMM entries (refine_select) for --shapes x --batch-sizes")
    args = ap.parse_args(list(argv) if argv is not None else None)
    if args.select:
        refine_select(args.shapes.split(","), [int(b) for b in args.batch_sizes.split(",")], table=args.table,
                      out_table=args.out, log=lambda m: print(m, flush=True))
        return
    if args.refine_kinds:
        refine(args.shapes.split(","), [int(b) for b in args.batch_sizes.split(",")],
               kinds=[int(v) for v in args.refine_kinds.split(",")], table=args.table, out_table=args.out,
               log=lambda m: print(m, flush=True))
        return
    shapes = {s: LLAMA2_7B_SHAPES[s] for s in args.shapes.split(",")}
    tune(shapes, [int(b) for b in args.batch_sizes.split(",")], [float(d) for d in args.densities.split(",")],
         out_table=args.out, lookup_dir=args.lookup_dir, log=lambda m: print(m, flush=True),
         merge_from=TABLE_PATH if args.merge else None)


if __name__ == "__main__":
    main()
