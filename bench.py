#!/usr/bin/env python3
"""Benchmark of the MI355X batch-shared block-sparse GEMM (one JSON line on stdout).

Default workload (the configuration the headline metric is quoted on):
every Llama-2-7B decoder projection shape -- q/k/v/o (K=4096 -> N=4096), gate/up (4096 -> 11008),
down (11008 -> 4096) -- at B=2 with block sparsity 0.803, B=16 at 0.638 and B=64 at 0.520, fp16,
each beside the same kernel with every block active (the in-run dense baseline).  The down_proj
B=16 sparsity sweep of configs[1] ({0, 0.25, 0.5, 0.638, 0.8}) rides along as extra points; its
s=0.5 point is the CPU-reference configuration of configs[0].

Rotation: one pool of packed-weight copies per projection shape.  A point's graph holds R
back-to-back launches, launch i reading copy i, with R = ceil(1 GiB / the point's ACTIVE weight
bytes), so every replay streams at least 1 GiB of distinct active weight and the 256 MB Infinity
Cache cannot serve a repeat.  A "step" is one replay of a graph holding every point's R launches.

value        = active-weight bytes of all GEMMs in the timed steps / timed seconds (GB/s)
roofline     = the dominant kernel (largest share of a step's GPU time, `by_kernel`) at its
               largest sparse launch (gate/up B=64 s=0.52 with the shipped plans): algorithmic
               bytes na*64*N*2 per launch over the average launch duration, from HIP events on the
               launch stream around that point's graph replays; the CPU-reference configuration
               (down_proj B=16 s=0.5) rides along as roofline.cpu_reference_point
cpu_baseline = the oracle's CPU path (torch CPU gather + fp32 matmul, every host core) on the
               configs[0] point, down_proj B=16 with 86 of 172 blocks; every point also carries
               its own CPU time

The same line also carries, measured in the same run after the matrix (skip with --no-extras):
fused_select_gemm = configs[3] (exact-L1 select k=31 of 64 + gate/up GEMM at B=64, indices
checked bit-exact), fused_select_gemm_b2 = the same call at q/k/v/o B=2 k=32 (one launch: the
GEMM scores the blocks itself), rule_select_gemm = the reference's decode linear with its own
selection rule (L2 mean, RRD:179-284) as one library call, beside its torch selection and in eager
calls of the model patch, decode_step = configs[4] (the 32-layer decode step of linears as one
hipGraph), eager_calls = the host cost of one eager call of the drop-in entry points (what
the model patch pays per linear layer), perstep_replay = the reference's headline table (its
per-step sparsity maps of the 224-GEMM decode step) at B=2, 4, 8, 16, 32, 64.

    python bench.py [--steps K] [--warmup W]
                    [--workload llama|down_sweep|fused|rule|decode|perstep|2d] [--only POINT]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(ROOT, "towards-batched-activation-sparsity_amd")
for _p in (PKG_ROOT, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 1 << 30
SEED = 1234
METRIC = "µs/GEMM + HBM GB/s + speedup vs dense, Llama-2-7B shapes at B=2/16/64"
# (K, N) of the Llama-2-7B projection shapes and the input distribution of each
SHAPES = {"qkvo": (4096, 4096), "gate_up": (4096, 11008), "down": (11008, 4096)}
X_DIST = {"qkvo": "normal", "gate_up": "normal", "down": "laplace"}
# Committed PMC summaries (HBM bytes per launch) of the roofline point of each workload.
TRAFFIC_PROFILES = {
    "down_b16_s500": os.path.join(ROOT, "profiles", "traffic_bsg_gemm_down_b16_s500.md"),
    "gate_up_b16_s638": os.path.join(ROOT, "profiles", "traffic_bsg_gemm_vt_gate_up_b16_s638.md"),
    "gate_up_b64_s520": os.path.join(ROOT, "profiles", "traffic_bsg_gemm_vtx_gate_up_b64_s520.md"),
}
# MFMA utilisation from counters (SQ_VALU_MFMA_BUSY_CYCLES) of the roofline point's kernel.
MFMA_PROFILES = {
    "down_b16_s500": os.path.join(ROOT, "profiles", "pmc_lds_mfma_bsg_gemm_down_b16_s500.md"),
    "gate_up_b16_s638": os.path.join(ROOT, "profiles", "pmc_lds_mfma_bsg_gemm_gate_up_b16_s638.md"),
    "gate_up_b64_s520": os.path.join(ROOT, "profiles", "pmc_lds_mfma_bsg_gemm_gate_up_b64_s520.md"),
}
# Kernel (symbol prefix) that each plan kind launches.
KERNEL_NAMES = {1: "bsg_gemm_kernel", 2: "bsg_gemm_xl_kernel", 3: "bsg_gemm_fma_kernel", 4: "bsg_gemm_xl_kernel",
                5: "bsg_gemm_vt_kernel", 6: "bsg_gemm_vt_kernel", 7: "bsg_gemm_vtx_kernel"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="llama",
                    choices=["llama", "down_sweep", "fused", "rule", "decode", "perstep", "2d", "timeline"])
    ap.add_argument("--plan", default=None,
                    help="timeline workload, or llama/down_sweep with --only: explicit plan a,b,c,d,e,f "
                         "(default: tuned)")
    ap.add_argument("--select", action="store_true",
                    help="timeline workload: the exact-L1 selection + GEMM (k = the point's blocks); stamps "
                         "cover the GEMM launch")
    ap.add_argument("--batches", default=None, help="perstep workload: batch sizes (default: all six)")
    ap.add_argument("--layers", type=int, default=32, help="decode workload: number of layers")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="llama workload: skip the configs[3] / configs[4] / per-step replay measurements that "
                         "the default line carries")
    ap.add_argument("--only", default=None, help="time only this point (profiling runs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the GEMMs, replay a plain device copy of MIB MiB (PMC calibration)")
    return ap.parse_args()


def copies_for(active_bytes: int) -> int:
    """Launches per graph so that one replay reads >= ROTATE_BYTES of distinct active weight."""
    return max(1, math.ceil(ROTATE_BYTES / max(1, int(active_bytes))))


class ShapePool:
    """Packed-weight copies of one projection shape.  W is the first draw of
    numpy default_rng(seed) -- N(0, 0.02) stored [K, N], fp16 -- exactly as oracle.make_inputs
    draws it, so every point of this shape sees the same W as its oracle inputs."""

    def __init__(self, name, k, n, dev, copies, seed=SEED):
        import numpy as np
        import torch

        import bsa_mi355x as bsa

        self.name, self.k, self.n, self.dev = name, k, n, dev
        self.nblk = (k + 63) // 64
        rng = np.random.default_rng(seed)
        self.w_kn_np = rng.normal(0.0, 0.02, size=(k, n)).astype(np.float16)
        w0 = torch.from_numpy(self.w_kn_np).to(dev)
        p0 = bsa.pack_weight(w0, layout="kn")
        del w0
        self.copies = max(1, int(copies))
        self.packed = [p0] + [p0.clone() for _ in range(self.copies - 1)]
        self.packed_bytes = p0.numel() * p0.element_size()
        self._kn = None

    def w_kn(self, count):
        """`count` [K, N] copies of W (hipBLASLt context), made on first use."""
        import torch

        if self._kn is None or len(self._kn) < count:
            w0 = torch.from_numpy(self.w_kn_np).to(self.dev)
            self._kn = [w0] + [w0.clone() for _ in range(count - 1)]
        return self._kn[:count]


class Point:
    """One GEMM configuration on a shape pool: its inputs, plan and a graph of R rotated launches."""

    def __init__(self, name, pool, bt, na, dev, dense=False, plan=None, inputs=None, seed=SEED):
        import torch

        import bsa_mi355x as bsa
        from oracle import bsg_oracle as orc

        self.name, self.pool, self.bt, self.dense = name, pool, bt, dense
        self.k, self.n, self.nblk = pool.k, pool.n, pool.nblk
        self.na = pool.nblk if dense else na
        if inputs is None:
            # x, then the mask, from oracle.make_inputs' rng stream (W is drawn first, as the pool's)
            x, _, idx = orc.make_inputs(seed, bt, self.k, self.n, X_DIST[pool.name], na=self.na)
        else:
            x, idx = inputs
        self.x_np, self.idx_np = x, idx
        self.x = torch.from_numpy(x).to(dev)
        self.idx = torch.from_numpy(idx).to(dev)
        self.y = torch.empty(bt, self.n, dtype=torch.float16, device=dev)
        self.plan = bsa.resolve_plan(bt, self.n, self.nblk, self.na, dev, plan, dense=dense)
        self.active_bytes = self.na * 64 * self.n * 2
        self.flops = 2 * bt * self.na * 64 * self.n
        self.copies = min(pool.copies, copies_for(self.active_bytes))
        self.graph = None
        self.in_step = True  # part of the timed step graph (comparison points are timed alone)

    @property
    def replay_bytes(self) -> int:
        return self.active_bytes * self.copies

    def launch(self, i):
        import bsa_mi355x as bsa

        p = self.pool.packed[i % self.copies]
        bsa.gemm_packed(self.x, p, self.n, None if self.dense else self.idx, self.y, plan=self.plan,
                        workspace_prefix=f"bench_{self.name}")

    def capture(self):
        self.graph = _capture([lambda i=i: self.launch(i) for i in range(self.copies)])

    def check(self):
        """Parity of the benchmarked launch against the oracle (fp32 CPU path)."""
        import numpy as np
        import torch

        from oracle import bsg_oracle as orc

        self.launch(0)
        torch.cuda.synchronize()
        w_nk = np.ascontiguousarray(self.pool.w_kn_np.T)
        ref = orc.gemm_ref(self.x_np, w_nk, self.idx_np)
        y = self.y.float().cpu().numpy()
        return orc.rel_frobenius(y, ref), orc.within_tolerance(y, ref)


def _capture(fns):
    """Warm up fns on a side stream (workspaces, plans), then capture them back to back as one graph."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    return g


def capture_step(points):
    """One hipGraph holding a whole step: every point's R rotated launches, back to back."""
    return _capture([lambda p=p, i=i: p.launch(i) for p in points for i in range(p.copies)])


def time_points(points, step_graph, steps, warmup, reps=10):
    """Warm-up, then exactly `steps` replays of the step graph between a synchronize + event
    pair on each side (the timed region); then each point's own graph, `reps` replays with a
    HIP-event pair on the launch stream around each, for the per-GEMM times."""
    import torch

    for _ in range(warmup):
        step_graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start_all = torch.cuda.Event(enable_timing=True)
    end_all = torch.cuda.Event(enable_timing=True)
    start_all.record()
    for _ in range(steps):
        step_graph.replay()
    end_all.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start_all.elapsed_time(end_all)
    per = {}
    for p in points:
        p.graph.replay()
        torch.cuda.synchronize()
        us = []
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            p.graph.replay()
            b.record()
            b.synchronize()
            us.append(a.elapsed_time(b) * 1000.0 / p.copies)
        per[p.name] = (statistics.median(us), statistics.mean(us))
    return total_ms, wall, per


def _cpu_tensors(point):
    import torch

    x = torch.from_numpy(point.x_np)
    w = torch.from_numpy(point.pool.w_kn_np)
    idx = torch.from_numpy(point.idx_np.astype("int64"))
    return x, w, idx


def cpu_baseline(point, seconds):
    """The oracle's CPU path on the GPU box's host cores: gather + convert + fp32 matmul, and the
    matmul alone on already gathered fp32 operands, each timed for about `seconds`."""
    import torch

    from oracle import bsg_oracle as orc

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x, w, idx = _cpu_tensors(point)

    def sample(fn, budget):
        for _ in range(2):
            fn()
        out = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end and len(out) < 500:
            t = time.perf_counter_ns()
            fn()
            out.append((time.perf_counter_ns() - t) / 1e3)
        return out

    full = sample(lambda: orc.gemm_ref_torch(x, w, idx), seconds * 0.7)
    cols = (64 * idx[:, None] + torch.arange(64)[None, :]).reshape(-1)
    xa = x.index_select(1, cols).float()
    wa = w.index_select(0, cols).float()
    mm = sample(lambda: xa @ wa, seconds * 0.3)
    us = statistics.median(full)
    us_mm = statistics.median(mm)
    return {
        "value": round(point.active_bytes / (us * 1e-6) / 1e9, 2),
        "unit": "GB/s",
        "us_per_gemm": round(us, 1),
        "matmul_only": {"us_per_gemm": round(us_mm, 1),
                        "GBps": round(point.active_bytes / (us_mm * 1e-6) / 1e9, 2), "runs": len(mm)},
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle gemm_ref_torch (torch CPU gather + fp32 matmul) on {point.name}: B={point.bt} "
                   f"K={point.k} N={point.n} {point.na}/{point.nblk} blocks; {len(full)} timed runs after 2 "
                   f"warm-ups, median; matmul_only = the fp32 matmul on pre-gathered operands"),
    }


def cpu_select_gemm_us(x_np, w_kn_np, keep, runs=3):
    """The CPU path of a select + GEMM (the oracle's exact-L1 top-k, then torch CPU gather + fp32
    matmul, every host core): the median of a few runs after one warm-up."""
    import torch

    from oracle import bsg_oracle as orc

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    x = torch.from_numpy(x_np)
    w = torch.from_numpy(w_kn_np)

    def run():
        idx = torch.from_numpy(orc.select_topk_l1(x_np, keep).astype("int64"))
        return orc.gemm_ref_torch(x, w, idx)

    run()
    samples = []
    for _ in range(runs):
        t = time.perf_counter_ns()
        run()
        samples.append((time.perf_counter_ns() - t) / 1e3)
    return statistics.median(samples)


def cpu_point_us(point, runs=5):
    """The same op on the oracle's CPU path (torch CPU gather + fp32 matmul, every host core): the
    median of a few runs after one warm-up, shown beside each point's GPU time."""
    import torch

    from oracle import bsg_oracle as orc

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    x, w, idx = _cpu_tensors(point)
    orc.gemm_ref_torch(x, w, idx)
    samples = []
    for _ in range(runs):
        t = time.perf_counter_ns()
        orc.gemm_ref_torch(x, w, idx)
        samples.append((time.perf_counter_ns() - t) / 1e3)
    return statistics.median(samples)


def _profile_value(path, key, conv):
    """The `key: value` line of a committed profile summary, or None."""
    if path is None:
        return None
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith(key + ":"):
                    return conv(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def load_mfma_util(point):
    """Counter-measured MFMA utilisation of a roofline point's kernel (committed PMC summary)."""
    path = MFMA_PROFILES.get(point)
    v = _profile_value(path, "mfma_util_counter", float)
    return None if v is None else {"value": v, "profile": os.path.relpath(path, ROOT)}


def load_traffic(point):
    """HBM bytes per launch of a roofline point, from its committed PMC summary (a line
    `traffic_bytes_per_launch: <int>`), or None when that point has no summary."""
    return _profile_value(TRAFFIC_PROFILES.get(point), "traffic_bytes_per_launch", int)


def copy_calibration(mib, steps):
    """Replay a plain device-to-device copy of `mib` MiB (known bytes) for PMC scaling."""
    import torch

    n = mib * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    g = torch.cuda.CUDAGraph()
    dst.copy_(src)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        dst.copy_(src)
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 2, "bytes_written": n * 2, "launches": steps + 1}))


def torch_mm_us(point, reps=5):
    """hipBLASLt dense GEMM (torch.mm) on the same shape, rotated over [K, N] weight copies
    (>= 1 GiB per replay): context for the dense points."""
    import torch

    ws = point.pool.w_kn(copies_for(point.pool.packed_bytes))
    out = torch.empty(point.bt, point.n, dtype=torch.float16, device=point.x.device)
    med, _ = _graph_time([lambda w=w: torch.mm(point.x, w, out=out) for w in ws], reps)
    return med / len(ws)


def read_calibration_us(point, reps=5):
    """Practical HBM read time of one launch streaming the point's active-weight bytes: the
    library's read-rate calibration kernel (the GEMM's weight-load pattern, no compute),
    rotated over the same weight copies and timed the same way."""
    import torch

    import bsa_mi355x as bsa

    lib = bsa.load()
    nbytes = point.active_bytes // 1024 * 1024
    sink = torch.zeros(4, dtype=torch.int32, device=point.x.device)

    def launch(i):
        def f():
            rc = lib.bsg_read_calibrate(point.pool.packed[i].data_ptr(), nbytes, sink.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(lib.bsg_last_error().decode())
        return f

    med, _ = _graph_time([launch(i) for i in range(point.copies)], reps)
    return med / point.copies


def _graph_time(fns, reps, warmup=2):
    """Capture fns back to back as one graph; median and mean µs per replay over `reps` replays."""
    import torch

    g = _capture(fns)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1000.0)
    del g
    return statistics.median(ts), statistics.mean(ts)


def sname(s: float) -> str:
    return f"s{int(round(s * 1000)):03d}"


# Suffix of the comparison points that run a B=2 sparse point on the dot-product kernel (kind 3,
# fp32 dot products with DPP quad sums) instead of the table's MFMA plan.
FMA_SUFFIX = "_fma"


def matrix_points(workload, dev):
    """The points of the llama (configs[2] + the configs[1] sweep) or down_sweep workload:
    [(name, shape, B, na, dense)].  The llama workload also holds, for each B=2 sparse point, a
    twin named <point>_fma on the dot-product kernel (timed on its own graph, outside the step)."""
    from oracle import bsg_oracle as orc

    rows = []
    if workload == "llama":
        for bt, s in ((2, 0.803), (16, 0.638), (64, 0.520)):
            for sh, (k, _) in SHAPES.items():
                nb = orc.nblk_of(k)
                rows.append((f"{sh}_b{bt}_{sname(s)}", sh, bt, orc.n_active_for_sparsity(s, nb), False))
                rows.append((f"{sh}_b{bt}_dense", sh, bt, nb, True))
    # down_proj B=16 over {0, 0.25, 0.5, 0.638, 0.8} (0.638 and 0 are in configs[2])
    have = {r[0] for r in rows}
    nb = orc.nblk_of(SHAPES["down"][0])
    for s in (0.0, 0.25, 0.5, 0.638, 0.8):
        name = "down_b16_dense" if s == 0.0 else f"down_b16_{sname(s)}"
        if name not in have:
            rows.append((name, "down", 16, nb if s == 0.0 else orc.n_active_for_sparsity(s, nb), s == 0.0))
    if workload == "llama":
        rows += [(r[0] + FMA_SUFFIX,) + r[1:] for r in list(rows) if r[2] == 2 and not r[4]]
    return rows


def pool_copies(rows):
    """Copies of each shape's packed weight: enough for its point with the fewest active bytes
    to read >= ROTATE_BYTES of distinct weight per replay (every other point uses a prefix)."""
    need = {}
    for _, sh, _, na, _ in rows:
        need[sh] = max(need.get(sh, 1), copies_for(na * 64 * SHAPES[sh][1] * 2))
    return need


def best_fma_plan(pool, bt, na, dev, inputs, reps=3):
    """The fastest dot-product (kind 3) plan for a point, each candidate the tuner would try
    (every instantiated kind-3 tile for the batch) timed on the point's own rotated graph."""
    import bsa_mi355x as bsa
    from bsa_mi355x import tuning

    best = None
    for cand in tuning.candidate_plans(bt, na, pool.nblk):
        if cand.kind != 3:
            continue
        try:
            pt = Point("fma_probe", pool, bt, na, dev, plan=cand, inputs=inputs)
        except (RuntimeError, ValueError):
            continue  # a tile whose activation staging cannot hold this list
        if pt.plan.kind != 3:
            continue
        med, _ = _graph_time([lambda i=i: pt.launch(i) for i in range(pt.copies)], reps)
        us = med / pt.copies
        if best is None or us < best[0]:
            best = (us, bsa.Plan(*pt.plan.as_tuple()))
    return None if best is None else best[1]


def run_matrix(args, dev):
    import torch

    rows = matrix_points(args.workload, dev)
    if args.only:
        rows = [r for r in rows if r[0] == args.only]
        if not rows:
            raise SystemExit(f"--only {args.only}: no such point")
    need = pool_copies(rows)
    pools = {sh: ShapePool(sh, *SHAPES[sh], dev, need[sh]) for sh in need}
    log("weight pools: " + ", ".join(f"{p.name} x{p.copies} ({p.copies * p.packed_bytes / 1e9:.1f} GB)"
                                     for p in pools.values()))
    # X once per (shape, B) and every mask of that pair from the same stream (oracle.make_inputs)
    from oracle import bsg_oracle as orc

    drawn = {}
    for key in dict.fromkeys((sh, bt) for _, sh, bt, _, _ in rows):
        nas = sorted({na for _, s2, b2, na, _ in rows if (s2, b2) == key})
        x, _, masks = orc.make_inputs(SEED, key[1], *SHAPES[key[0]], X_DIST[key[0]], na=nas)
        drawn[key] = (x, dict(zip(nas, masks)))
    forced = None
    if args.plan:
        if not args.only:
            raise SystemExit("--plan needs --only")
        import bsa_mi355x as bsa

        forced = bsa.Plan(*[int(v) for v in args.plan.split(",")])
    points = []
    for name, sh, bt, na, dense in rows:
        x, masks = drawn[(sh, bt)]
        plan = forced
        if name.endswith(FMA_SUFFIX) and forced is None:
            plan = best_fma_plan(pools[sh], bt, na, dev, (x, masks[na]))
            if plan is None:
                log(f"{name}: no dot-product tile runs this point; skipped")
                continue
        points.append(Point(name, pools[sh], bt, na, dev, dense=dense, plan=plan, inputs=(x, masks[na])))
        points[-1].in_step = not name.endswith(FMA_SUFFIX)
        log(f"prepared {name}: na={points[-1].na} copies={points[-1].copies} "
            f"replay={points[-1].replay_bytes / 2**30:.2f} GiB plan={points[-1].plan}")
    bad = []
    for p in points:
        rf, ok = p.check()
        if not ok:
            bad.append((p.name, rf))
    if bad:
        raise SystemExit(f"parity failure before timing: {bad}")
    log("parity ok on every point")
    for p in points:
        p.capture()
    step_points = [p for p in points if p.in_step]
    step_graph = capture_step(step_points)
    log("graphs captured")

    total_ms, wall, per = time_points(points, step_graph, args.steps, args.warmup)
    step_bytes = sum(p.replay_bytes for p in step_points)
    value = step_bytes * args.steps / (total_ms * 1e-3) / 1e9
    log(f"timed {args.steps} steps in {total_ms:.2f} ms (host wall {wall * 1e3:.1f} ms)")

    dense_us = {p.name[: -len("_dense")]: per[p.name][0] for p in points if p.dense}
    out_points = []
    for p in points:
        med, mean = per[p.name]
        gbs = p.active_bytes / (med * 1e-6) / 1e9
        row = {"name": p.name, "B": p.bt, "K": p.k, "N": p.n, "active_blocks": p.na, "nblk": p.nblk,
               "us_per_gemm": round(med, 3), "GBps_active": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
               "floor_us_at_8TBps": round(p.active_bytes / (HBM_PEAK_GBS * 1e3), 3),
               "replay_GiB": round(p.replay_bytes / 2**30, 3), "plan": list(p.plan.as_tuple()),
               "kernel": KERNEL_NAMES.get(p.plan.kind, "bsg_gemm")}
        if p.bt >= 16:
            # derived (flops / time / peak), not a counter reading
            row["mfma_util_derived"] = round(p.flops / (med * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 5)
        if not p.dense:
            d = dense_us.get(p.name.rsplit("_s", 1)[0])
            if d:
                row["speedup_vs_dense"] = round(d / med, 3)
                row["ideal_speedup"] = round(p.nblk / p.na, 3)
                row["speedup_over_ideal"] = round((d / med) / (p.nblk / p.na), 3)
        if p.name.endswith(FMA_SUFFIX):
            twin = p.name[: -len(FMA_SUFFIX)]
            row["in_step"] = False
            row["mfma_point"] = twin
            row["mfma_us_per_gemm"] = round(per[twin][0], 3)
            row["fma_over_mfma_time"] = round(med / per[twin][0], 3)
        if not args.only:
            # the practical read of the same bytes per launch (same rotation and timing)
            rd = read_calibration_us(p)
            row["practical_read_us"] = round(rd, 3)
            row["frac_of_practical_read"] = round(rd / med, 4)
        out_points.append(row)
        log(json.dumps(row))

    shares = kernel_shares(step_points, per)
    focus = roofline_point(step_points, shares) if not args.only else points[0].name

    def roofline_of(name, with_read):
        fp = next(p for p in points if p.name == name)
        f_med, f_mean = per[name]
        achieved = fp.active_bytes / (f_mean * 1e-6) / 1e9
        r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
             "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic(name),
             "kernel": KERNEL_NAMES.get(fp.plan.kind, "bsg_gemm"), "point": name,
             "avg_launch_us": round(f_mean, 3), "bytes_per_launch": fp.active_bytes,
             "plan": list(fp.plan.as_tuple())}
        mf = load_mfma_util(name)
        if mf is not None:
            r["mfma_util_counter"] = mf
        if with_read:
            rd = read_calibration_us(fp)
            r["practical_read"] = {
                "us_per_launch": round(rd, 3), "GBps": round(fp.active_bytes / (rd * 1e-6) / 1e9, 1),
                "frac_of_it": round(rd / f_mean, 4),
                "what": "bsg_read_calibrate streaming the same bytes per launch (weight-load pattern, no compute), "
                        "same rotation and timing"}
            log(f"practical read of {fp.active_bytes / 1e6:.2f} MB: {rd:.2f} us ({r['practical_read']['GBps']} GB/s)")
        return r

    roofline = roofline_of(focus, not args.only)
    roofline["chosen_as"] = ("the dominant kernel (largest share of the step's GPU time, by_kernel) at its "
                             "largest sparse launch" if not args.only else "the --only point")
    roofline["by_kernel"] = shares
    if not args.only and focus != "down_b16_s500" and any(p.name == "down_b16_s500" for p in points):
        # the CPU-reference configuration beside it
        roofline["cpu_reference_point"] = roofline_of("down_b16_s500", True)
    if not args.only and focus != "gate_up_b64_s520" and any(p.name == "gate_up_b64_s520" for p in points):
        # configs[3]'s GEMM (gate/up B=64, 31 of 64 blocks), whichever kernel runs it
        roofline["configs3_gemm_point"] = roofline_of("gate_up_b64_s520", True)
    if not args.only:
        # hipBLASLt (torch.mm, the reference's dense baseline) beside every dense point, so the
        # dense kernel the speedups divide by is shown against the vendor library at each batch
        for p, row in zip(points, out_points):
            if p.dense:
                row["torch_mm_us"] = round(torch_mm_us(p), 3)
                log(f"torch.mm (hipBLASLt) on {p.name}: {row['torch_mm_us']:.2f} us")
    extras = {}
    if args.workload == "llama" and not args.only and not args.no_extras:
        # BASELINE configs[3] and configs[4] and the reference's headline table, measured in the
        # same run; the matrix's weight pools and graphs are released first
        for p in points:
            p.graph = None
        step_graph = None
        for pool in pools.values():  # the CPU baseline below needs only the pools' host copies
            pool.packed = []
            pool._kn = None
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        log("configs[3]: fused exact-L1 select + GEMM ...")
        extras["fused_select_gemm"] = measure_fused(args, dev)
        log(f"configs[3] done ({time.perf_counter() - t0:.1f} s): {extras['fused_select_gemm']['us_select_plus_gemm']} us")
        extras["fused_select_gemm_b2"] = measure_fused(args, dev, shape="qkvo", bt=2, keep=32)
        log(f"select + GEMM at q/k/v/o B=2: {extras['fused_select_gemm_b2']['us_select_plus_gemm']} us "
            f"(GEMM alone {extras['fused_select_gemm_b2']['us_gemm_only']} us)")
        log("the reference's decode linear (its selection rule) as one call ...")
        extras["rule_select_gemm"] = measure_rule_linear(args, dev)
        log(f"reference-rule select + GEMM: {extras['rule_select_gemm']['us_fused_rule_select_gemm']} us fused, "
            f"{extras['rule_select_gemm']['us_reference_torch_select_then_gemm']} us with the reference's torch "
            f"selection (GEMM alone {extras['rule_select_gemm']['us_gemm_only']} us)")
        log("configs[4]: 32-layer decode step ...")
        extras["decode_step"] = measure_decode(args, dev)
        log(f"configs[4] done ({time.perf_counter() - t0:.1f} s): {extras['decode_step']['ms_per_step']} ms/step")
        log("eager host cost of the drop-in entry points ...")
        extras["eager_calls"] = measure_eager(args, dev)
        log("per-step replay of the reference's sparsity maps at every batch size ...")
        rows_ps, _, _ = measure_perstep(args, dev)
        extras["perstep_replay"] = {
            "workload": "the reference's headline table (scripts/bench_perstep_actual_kernel_speedup.py, "
                        "README.md:32-36): its per-step sparsity maps of the 224-GEMM decode step replayed on this "
                        "build at B=2..64; speedup of the sparse step over our own dense kernel and over "
                        "hipBLASLt, beside the reference's A100X speedup over cuBLAS",
            "rows": [{k: r[k] for k in ("B", "group_steps", "mean_sparsity", "speedup_vs_own_dense",
                                        "speedup_vs_hipblaslt", "reference_a100x_speedup_vs_cublas",
                                        "sparse_us_step_mean", "replay_tokens_per_s",
                                        "reference_a100x_replay_tokens_per_s")} for r in rows_ps]}
        log("each group-step as one 224-GEMM graph ...")
        extras["perstep_replay"]["step_graphs"] = measure_step_graphs(args, dev)
        log(f"extras done ({time.perf_counter() - t0:.1f} s)")
    cpu = None
    if not args.no_cpu and not args.only:
        log("cpu baseline ...")
        cpu_pt = next((p for p in points if p.name == "down_b16_s500"), next(p for p in points if p.name == focus))
        cpu = cpu_baseline(cpu_pt, args.cpu_seconds)
        for p, row in zip(points, out_points):
            row["cpu_us_per_gemm"] = round(cpu_point_us(p), 1)
            row["gpu_speedup_over_cpu"] = round(row["cpu_us_per_gemm"] / row["us_per_gemm"], 1)
    sparse = [r for r in out_points if "speedup_over_ideal" in r and r.get("in_step", True)]
    fma_rows = [r for r in out_points if not r.get("in_step", True)]
    if args.workload == "llama":
        workload = ("Llama-2-7B q/k/v/o (4096->4096), gate/up (4096->11008), down (11008->4096) at B=2@0.803, "
                    "B=16@0.638, B=64@0.520, each with its dense point (configs[2]); plus the down_proj B=16 "
                    "sweep {0,0.25,0.5,0.638,0.8} (configs[1])")
    else:
        workload = "down_proj B=16 K=11008 N=4096 fp16, block sparsity sweep {0,0.25,0.5,0.638,0.8} (configs[1])"
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: numpy PCG64 seed 1234, W~N(0,0.02) stored [K,N], X~Laplace(0,0.05) (down) / N(0,1) "
                "(others), masks rng.choice sorted; each point's graph rotates over >=1 GiB of distinct active "
                "weight",
        "config": {"workload": workload, "gemms_per_step": sum(p.copies for p in step_points),
                   "value_is": "active-weight bytes / timed seconds over all points of the step (the "
                               "dot-product comparison points are timed on their own graphs, outside it)",
                   "min_replay_GiB": round(min(p.replay_bytes for p in points) / 2**30, 3)},
        "points": out_points,
        "summary": {
            "sparse_points": len(sparse),
            "mean_frac_hbm_peak_sparse": round(statistics.mean(r["frac_hbm_peak"] for r in sparse), 4) if sparse else None,
            "mean_speedup_over_ideal": round(statistics.mean(r["speedup_over_ideal"] for r in sparse), 4) if sparse else None,
            "mean_frac_of_practical_read": round(statistics.mean(r["frac_of_practical_read"] for r in out_points
                                                                 if "frac_of_practical_read" in r), 4)
            if any("frac_of_practical_read" in r for r in out_points) else None,
            "b64_frac_of_practical_read": {r["name"]: r["frac_of_practical_read"] for r in out_points
                                           if r["B"] == 64 and "frac_of_practical_read" in r},
            "dot_product_vs_mfma_at_b2": {r["mfma_point"]: {"fma_us": r["us_per_gemm"], "mfma_us": r["mfma_us_per_gemm"],
                                                             "fma_plan": r["plan"]} for r in fma_rows},
            "dense_vs_hipblaslt": {r["name"]: {"own_us": r["us_per_gemm"], "hipblaslt_us": r["torch_mm_us"],
                                               "own_speedup": round(r["torch_mm_us"] / r["us_per_gemm"], 3)}
                                   for r in out_points if "torch_mm_us" in r},
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    line.update(extras)
    print(json.dumps(line), flush=True)


def roofline_point(points, shares):
    """The roofline point: the dominant kernel (largest share of the step's GPU time) at its
    largest sparse launch (most active-weight bytes per launch, a streaming launch rather than a
    latency-bound one); the dominant kernel's largest launch of any kind when it runs no sparse
    point."""
    dominant = next(iter(shares))  # kernel_shares orders by time share
    mine = [p for p in points if KERNEL_NAMES.get(p.plan.kind, "bsg_gemm") == dominant]
    sparse = [p for p in mine if not getattr(p, "dense", False)] or mine
    return max(sparse, key=lambda p: (p.active_bytes, p.name)).name


def kernel_shares(points, per):
    """Per kernel (symbol prefix of the plans' kinds): its share of one step's GPU time (each point
    weighted by its launches per step), and active-weight bytes over that time against the peak."""
    acc = {}
    for p in points:
        name = KERNEL_NAMES.get(p.plan.kind, "bsg_gemm")
        us = per[p.name][1] * p.copies
        a = acc.setdefault(name, {"us": 0.0, "bytes": 0, "points": [], "top": (0.0, None)})
        a["us"] += us
        a["bytes"] += p.active_bytes * p.copies
        a["points"].append(p.name)
        if us > a["top"][0]:
            a["top"] = (us, p.name)
    total = sum(a["us"] for a in acc.values())
    out = {}
    for name, a in sorted(acc.items(), key=lambda kv: -kv[1]["us"]):
        gbs = a["bytes"] / (a["us"] * 1e-6) / 1e9
        out[name] = {"time_share": round(a["us"] / total, 4), "GBps": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "points": a["points"], "top_point": a["top"][1]}
    return out


def run_2d(args, dev):
    """2-D block sparsity (active output blocks as well as K-blocks): down_proj B=16 with half of the K-blocks
    active and a sweep of active 64-column output blocks, in place and compact.  Each point is
    a graph of launches rotated over >= 1 GiB of distinct active weight; parity against the
    oracle first.  Bytes per launch: na * 64 * (nn * 64) * 2 (active weight)."""
    import numpy as np
    import torch

    from bsa_mi355x import sparse2d
    from oracle import bsg_oracle as orc

    bt, k, n = 16, 11008, 4096
    nb_k, nb_n = orc.nblk_of(k), n // 64
    na = orc.n_active_for_sparsity(0.5, nb_k)
    x, _, kidx = orc.make_inputs(SEED, bt, k, n, "laplace", na=na)
    sweep = ((1.0, False), (0.75, False), (0.5, False), (0.25, False), (0.5, True))
    min_nn = min(int(round(nd * nb_n)) for nd, _ in sweep)
    pool = ShapePool("down", k, n, dev, copies_for(na * 64 * min_nn * 64 * 2))
    rng = np.random.default_rng(4321)
    xt, kt = torch.from_numpy(x).to(dev), torch.from_numpy(kidx).to(dev)
    w_nk = np.ascontiguousarray(pool.w_kn_np.T)
    reps = max(5, args.steps)
    rows, total_bytes, total_us, focus = [], 0, 0.0, None
    for nd, compact in sweep:
        nn = int(round(nd * nb_n))
        nidx = np.sort(rng.choice(nb_n, nn, replace=False)).astype(np.int32)
        nt = torch.from_numpy(nidx).to(dev)
        y = torch.zeros(bt, nn * 64 if compact else n, dtype=torch.float16, device=dev)
        pl = sparse2d.plan_2d(bt, n, nn, nb_k, len(kidx), dev)
        b = len(kidx) * 64 * nn * 64 * 2
        copies = min(pool.copies, copies_for(b))

        def call(i, nt=nt, y=y, compact=compact, pl=pl):
            return lambda: sparse2d.gemm_2d_packed(xt, pool.packed[i], n, kt, nt, y, compact=compact, plan=pl,
                                                   workspace_prefix="bench2d")

        call(0)()
        torch.cuda.synchronize()
        want = orc.gemm_2d_ref(x, w_nk, kidx, nidx, out_init=np.zeros((bt, n), np.float32), compact=compact)
        if not orc.within_tolerance(y.float().cpu().numpy(), want):
            raise SystemExit(f"2-D parity failure at n-density {nd} compact={compact}")
        med, mean = _graph_time([call(i) for i in range(copies)], reps)
        us, us_mean = med / copies, mean / copies
        total_bytes += b * copies
        total_us += med
        name = f"down_b16_k500_n{int(round(nd * 1000)):04d}{'_compact' if compact else ''}"
        row = {"name": name, "active_k_blocks": len(kidx), "active_n_blocks": nn, "compact": compact,
               "us_per_gemm": round(us, 3), "GBps_active": round(b / (us * 1e-6) / 1e9, 1),
               "replay_GiB": round(b * copies / 2**30, 3), "plan": list(pl.as_tuple())}
        rows.append(row)
        log(json.dumps(row))
        if nd == 0.5 and not compact:
            focus = (row, b, us_mean)
    full = rows[0]["us_per_gemm"]
    for r in rows[1:]:
        r["speedup_vs_all_n_blocks"] = round(full / r["us_per_gemm"], 3)
        r["ideal"] = round(nb_n / r["active_n_blocks"], 3)
    frow, fb, fmean = focus
    achieved = fb / (fmean * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(total_bytes / (total_us * 1e-6) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": reps, "warmup": 2, "ms_per_step": round(total_us / 1000.0, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: numpy PCG64 seed 1234 (X~Laplace(0,0.05), W~N(0,0.02)), K mask rng.choice of 86/172, "
                "output-block masks rng.choice seed 4321; each point rotates over >=1 GiB of distinct active weight",
        "config": {"workload": "2-D block sparsity: down_proj B=16 K=11008 N=4096, K density 0.5, output-block "
                               "density {1, 0.75, 0.5, 0.25} in place + 0.5 compact"},
        "points": rows,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "bsg_gemm_kernel (2-D)",
                     "point": frow["name"], "avg_launch_us": round(fmean, 3), "bytes_per_launch": fb},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def measure_eager(args, dev):
    """Host cost of one eager call of the drop-in entry points: no graph, what the reference's
    model patch pays per linear layer (RRD:228-230 calls the runtime entry per forward).  At
    down_proj B=16 s=0.5 with an unsorted list: host microseconds per call over back-to-back
    calls, and wall microseconds per call once the GPU has drained (the larger of the host's
    and the GPU's time per call).  The drop-in's output is checked against the oracle first."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from bsa_mi355x.select import select_gemm_packed
    from oracle import bsg_oracle as orc

    bt, (k, n), na, reps = 16, SHAPES["down"], 86, 2000
    g = torch.Generator(device=dev)
    g.manual_seed(SEED)
    x = torch.randn(bt, 1, k, generator=g, device=dev).to(torch.float16)
    w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.float16)
    ids = torch.randperm(k // 64, generator=g, device=dev)[:na].to(torch.int32)  # unsorted
    ids_sorted = torch.sort(ids)[0]
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    x2d, y2d = x.view(bt, k), out.view(bt, n)
    packed = bsa.pack_weight(w)
    wt = w.t().contiguous()
    idx = torch.empty(na, dtype=torch.int32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    bsa._prepacked_block_sparse_gemm_from_active_blocks(x, w, ids, out, cache_prefix="eager_bench")
    torch.cuda.synchronize()
    y_ref = orc.gemm_ref(x2d.float().cpu().numpy(), w.float().cpu().numpy(), ids_sorted.cpu().numpy())
    if not orc.within_tolerance(y2d.float().cpu().numpy(), y_ref):
        raise SystemExit("eager drop-in output outside tolerance")
    # fresh activation and output tensors per call (a decode loop's x and out are new each token)
    xs = [x.clone() for _ in range(4)]
    outs = [torch.empty_like(out) for _ in range(4)]
    turn = [0]

    def dropin_fresh():
        i = turn[0] = (turn[0] + 1) & 3
        bsa._prepacked_block_sparse_gemm_from_active_blocks(xs[i], w, ids, outs[i], cache_prefix="eager_bench")

    calls = {
        "dropin_unsorted_list": lambda: bsa._prepacked_block_sparse_gemm_from_active_blocks(
            x, w, ids, out, cache_prefix="eager_bench"),
        "dropin_fresh_x_and_out": dropin_fresh,
        "gemm_packed_table_plan": lambda: bsa.gemm_packed(x2d, packed, n, ids_sorted, y2d,
                                                          workspace_prefix="eager_bench_packed"),
        "select_gemm_packed": lambda: select_gemm_packed(x2d, packed, n, na, y2d, idx_out=idx, count_out=cnt,
                                                         workspace_prefix="eager_bench_sel"),
        "torch_mm_dense": lambda: torch.mm(x2d, wt, out=y2d),
    }
    res = {"workload": f"eager calls at down_proj B={bt} K={k} N={n}, {na}/{k // 64} blocks (s=0.5), "
                       f"unsorted list for the drop-in; {reps} back-to-back calls per entry",
           "what": "host_us = host time per call (Python + launch); wall_us = time per call until the GPU "
                   "has drained (the larger of host and GPU time per call)"}
    for name, fn in calls.items():
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        res[name] = {"host_us": round((t1 - t0) / reps * 1e6, 2), "wall_us": round((t2 - t0) / reps * 1e6, 2)}
        log(f"eager {name}: host {res[name]['host_us']} us/call, wall {res[name]['wall_us']} us/call")
    return res


def measure_fused(args, dev, shape="gate_up", bt=64, keep=31):
    """BASELINE config 4 (the defaults): fused exact-L1 selection (k=31 of 64) + sparse GEMM on
    gate/up at B=64 (K=4096 -> N=11008), rotated over >= 1 GiB of distinct active weight; indices
    checked bit-exact against the oracle first.  Other (shape, bt, keep) measure the same call
    elsewhere (at bt <= 8 and bt x K x 2 <= 24 KiB it is one launch).  Returns the measured
    fields."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from bsa_mi355x.select import select_gemm_packed
    from oracle import bsg_oracle as orc

    k, n = SHAPES[shape]
    pool = ShapePool(shape, k, n, dev, copies_for(keep * 64 * n * 2))
    pt = Point(f"{shape}_b{bt}_fused", pool, bt, keep, dev)
    idx = torch.empty(keep, dtype=torch.int32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    select_gemm_packed(pt.x, pool.packed[0], n, keep, pt.y, idx_out=idx, count_out=cnt, workspace_prefix="fused_bench")
    torch.cuda.synchronize()
    want = orc.select_topk_l1(pt.x_np, keep)
    got = idx.cpu().numpy()
    if not np.array_equal(got, want) or int(cnt.item()) != keep:
        raise SystemExit(f"fused selector indices differ from the oracle: {got} vs {want}")
    y_ref = orc.gemm_ref(pt.x_np, np.ascontiguousarray(pool.w_kn_np.T), want)
    if not orc.within_tolerance(pt.y.float().cpu().numpy(), y_ref):
        raise SystemExit("fused select+GEMM output outside tolerance")
    log("fused: indices bit-exact, GEMM within tolerance")
    # each call with its own tuned plan: the selection + GEMM entry, and the plain GEMM's
    plan = bsa.resolve_plan(bt, n, pt.nblk, keep, dev, select=True)
    plan_gemm = bsa.resolve_plan(bt, n, pt.nblk, keep, dev)

    def fused(i):
        return lambda: select_gemm_packed(pt.x, pool.packed[i], n, keep, pt.y, plan=plan, idx_out=idx, count_out=cnt,
                                          workspace_prefix="fused_bench")

    def gemm_only(i):
        return lambda: bsa.gemm_packed(pt.x, pool.packed[i], n, idx, pt.y, plan=plan_gemm,
                                       workspace_prefix="fused_gemm")

    def select_only(i):
        return lambda: bsa.select_topk_l1(pt.x, keep, idx_out=idx, count_out=cnt, workspace_prefix="fused_sel")

    r = pt.copies
    reps = max(5, args.steps)
    t_fused = _graph_time([fused(i) for i in range(r)], reps)[0] / r
    t_gemm = _graph_time([gemm_only(i) for i in range(r)], reps)[0] / r
    t_sel = _graph_time([select_only(i) for i in range(r)], reps)[0] / r
    gbs = pt.active_bytes / (t_fused * 1e-6) / 1e9
    cpu = {}
    if not args.no_cpu:
        cpu_us = cpu_select_gemm_us(pt.x_np, pool.w_kn_np, keep)
        cpu = {"cpu_us_select_plus_gemm": round(cpu_us, 1), "cpu_cores": len(os.sched_getaffinity(0)),
               "gpu_speedup_over_cpu": round(cpu_us / t_fused, 1)}
    out = {"workload": f"fused exact-L1 select (k={keep} of {pt.nblk}) + sparse GEMM, {shape} B={bt} K={k} N={n}"
                       + (" (configs[3])" if (shape, bt, keep) == ("gate_up", 64, 31) else
                          " (one launch: the GEMM scores the blocks itself)" if bt <= 8 and bt * k * 2 <= 24576 else ""),
           "us_select_plus_gemm": round(t_fused, 3), "us_gemm_only": round(t_gemm, 3),
           "us_select_only": round(t_sel, 3), "select_overhead_us": round(t_fused - t_gemm, 3),
           "GBps_active": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "plan": list(plan.as_tuple()), "plan_gemm_only": list(plan_gemm.as_tuple()), "launches_per_replay": r, "replays": reps, "indices_bit_exact": True,
           **cpu}
    del pool, pt
    torch.cuda.empty_cache()
    return out


def measure_rule_linear(args, dev, shape="gate_up", bt=64, density=0.48):
    """The reference's decode linear (`_sparse_linear`, RRD:179-284) on gate/up at B=64: its own
    selection rule (`_select_active_blocks`: batch-mean L2 norm, n_keep = round(0.48 x 64) = 31)
    then the GEMM.  Timed as graphs rotated over >= 1 GiB of active weight, three ways: one
    library call (bsg_select_gemm_rule: score launch + a GEMM that ranks the scores itself),
    the library's selector then the GEMM on its device count (three launches), and the
    reference's torch selection (norm, mean, topk, sort: its op chain, RRD:97-113) then the GEMM.
    Then eager calls of the model patch's `_sparse_linear` (what a decode step pays per linear),
    fused and with selection and GEMM as separate calls.  Ids are checked against the oracle
    (float64, select_scored_ref) first."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from bsa_mi355x import patch
    from bsa_mi355x.select import select_gemm_rule_packed
    from oracle import bsg_oracle as orc

    k, n = SHAPES[shape]
    nblk = k // 64
    keep = orc.n_keep(density, nblk)
    pool = ShapePool(shape, k, n, dev, copies_for(keep * 64 * n * 2))
    pt = Point(f"{shape}_b{bt}_rule", pool, bt, keep, dev)
    idx = torch.empty(keep, dtype=torch.int32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    select_gemm_rule_packed(pt.x, pool.packed[0], n, keep, pt.y, score="l2_mean", idx_out=idx, count_out=cnt,
                            workspace_prefix="rule_bench")
    torch.cuda.synchronize()
    want, _, _ = orc.select_scored_ref(pt.x_np, keep, "l2_mean")
    if not np.array_equal(idx.cpu().numpy(), want) or int(cnt.item()) != keep:
        raise SystemExit("reference-rule selection differs from the oracle")
    if not orc.within_tolerance(pt.y.float().cpu().numpy(),
                                orc.gemm_ref(pt.x_np, np.ascontiguousarray(pool.w_kn_np.T), want)):
        raise SystemExit("reference-rule select + GEMM output outside tolerance")
    plan = bsa.resolve_plan(bt, n, nblk, keep, dev, select=True)
    plan_gemm = bsa.resolve_plan(bt, n, nblk, keep, dev)
    x3 = pt.x.view(bt, 1, k)

    def fused(i):
        return lambda: select_gemm_rule_packed(pt.x, pool.packed[i], n, keep, pt.y, score="l2_mean", plan=plan,
                                               idx_out=idx, count_out=cnt, workspace_prefix="rule_bench")

    def separate(i):
        def f():
            bsa.select_topk(pt.x, keep, score="l2_mean", idx_out=idx, count_out=cnt, workspace_prefix="rule_sel")
            bsa.gemm_packed(pt.x, pool.packed[i], n, idx, pt.y, num_active=keep, num_active_dev=cnt, plan=plan_gemm,
                            workspace_prefix="rule_gemm")
        return f

    def torch_select(i):
        def f():
            xb = x3[..., : nblk * 64].float().reshape(-1, nblk, 64)
            sel = torch.topk(xb.norm(dim=2).mean(dim=0), k=keep).indices.sort()[0].to(torch.int32)
            bsa.gemm_packed(pt.x, pool.packed[i], n, sel, pt.y, num_active=keep, plan=plan_gemm,
                            workspace_prefix="rule_gemm_t")
        return f

    def gemm_only(i):
        return lambda: bsa.gemm_packed(pt.x, pool.packed[i], n, idx, pt.y, num_active=keep, plan=plan_gemm,
                                       workspace_prefix="rule_gemm")

    r = pt.copies
    reps = max(5, args.steps)
    t = {name: _graph_time([fn(i) for i in range(r)], reps)[0] / r
         for name, fn in (("fused", fused), ("separate", separate), ("torch_select", torch_select),
                          ("gemm_only", gemm_only))}
    # eager: the patched linear per call (a decode step calls it once per projection)
    w = torch.from_numpy(np.ascontiguousarray(pool.w_kn_np.T)).to(dev)
    cfg = {"best_kern": "naive", "best_K": 1, "best_tile": None}
    stats = {"calls": 0, "wall_s": 0.0}

    def eager_fused():
        patch._sparse_linear(x3, w, density, cfg, "rule_eager", 64, stats, False, None)

    def eager_separate():
        sel = bsa._select_active_blocks(x3, density, 64)
        out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
        bsa._prepacked_block_sparse_gemm_from_active_blocks(x3, w, sel, out, cache_prefix="rule_eager",
                                                            use_run_compressed=False)

    eager = {}
    for name, fn in (("patched_linear_fused", eager_fused), ("select_then_gemm_calls", eager_separate)):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        n_calls = 500
        t0 = time.perf_counter()
        for _ in range(n_calls):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        eager[name] = {"host_us": round((t1 - t0) / n_calls * 1e6, 2), "wall_us": round((t2 - t0) / n_calls * 1e6, 2)}
    out = {"workload": f"the reference's decode linear (L2-mean rule, k={keep} of {nblk}) + sparse GEMM, {shape} "
                       f"B={bt} K={k} N={n}: RRD:179-284 with _select_active_blocks",
           "us_fused_rule_select_gemm": round(t["fused"], 3),
           "us_library_select_then_gemm": round(t["separate"], 3),
           "us_reference_torch_select_then_gemm": round(t["torch_select"], 3),
           "us_gemm_only": round(t["gemm_only"], 3),
           "select_overhead_us_fused": round(t["fused"] - t["gemm_only"], 3),
           "select_overhead_us_reference_torch": round(t["torch_select"] - t["gemm_only"], 3),
           "plan": list(plan.as_tuple()), "plan_gemm_only": list(plan_gemm.as_tuple()), "indices_bit_exact": True,
           "eager": eager, "launches_per_replay": r, "replays": reps}
    del pool, pt, w
    torch.cuda.empty_cache()
    return out


def run_fused(args, dev):
    """`--workload fused`: the configs[3] measurement as its own JSON line."""
    f = measure_fused(args, dev)
    r, reps = f["launches_per_replay"], f["replays"]
    line = {
        "metric": METRIC, "value": f["GBps_active"], "unit": "GB/s", "n_gpus": 1, "steps": reps,
        "warmup": 2, "ms_per_step": round(f["us_select_plus_gemm"] * r / 1000.0, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: numpy PCG64 seed 1234, W~N(0,0.02) [K,N], X~N(0,1); >=1 GiB of distinct active weight "
                "per replay",
        "config": {"workload": f["workload"], "plan": f["plan"], "launches_per_replay": r},
        **{k: f[k] for k in ("us_select_plus_gemm", "us_gemm_only", "us_select_only", "select_overhead_us",
                             "indices_bit_exact")},
    }
    print(json.dumps(line), flush=True)


def measure_decode(args, dev):
    """Llama-2-7B-shaped decode step of linears (layers x {qkv, o, gate/up,
    down}), B=64, per-projection masks from the fused selector at density 0.48 (k=31/64, 83/172),
    the whole step captured as one hipGraph.  Its full parity check (every projection's indices,
    first and last layer outputs, replay against eager) is tests/test_gpu_decode.py; here the
    first and last layers are spot-checked before timing.  Returns the measured fields."""
    import numpy as np
    import torch

    from bsa_mi355x.decode import DecodeStep
    from oracle import bsg_oracle as orc

    t0 = time.perf_counter()
    step = DecodeStep(batch=64, density=0.48, n_layers=args.layers, device=dev)
    log(f"decode: {args.layers} layers, {step.resident_weight_bytes / 1e9:.2f} GB packed weights resident, "
        f"{step.active_bytes / 1e9:.3f} GB active per step ({time.perf_counter() - t0:.1f} s to build)")
    step.capture()
    torch.cuda.synchronize()
    cpu_layer_us = 0.0
    for li in sorted({0, args.layers - 1}):
        for p in step.layers[li]:
            x = p.x.cpu().numpy()
            want = orc.select_topk_l1(x, p.keep)
            got = p.idx[: min(p.keep, p.nblk)].cpu().numpy()
            if not np.array_equal(got, want):
                raise SystemExit(f"decode layer {li} {p.name}: selected blocks differ from the oracle")
            w_kn = np.ascontiguousarray(orc.tile_unpermute(p.packed.cpu().numpy(), p.n).reshape(-1, p.n)[: p.k])
            if not orc.within_tolerance(p.y.float().cpu().numpy(), orc.gemm_ref(x, np.ascontiguousarray(w_kn.T), want)):
                raise SystemExit(f"decode layer {li} {p.name}: output outside tolerance")
            if li == 0 and not args.no_cpu:
                cpu_layer_us += cpu_select_gemm_us(x, w_kn, p.keep, runs=1)
    log("decode: parity ok (first/last layer, all projections)")
    for _ in range(args.warmup):
        step.replay()
    torch.cuda.synchronize()
    ts = []
    a0 = torch.cuda.Event(enable_timing=True)
    b0 = torch.cuda.Event(enable_timing=True)
    a0.record()
    for _ in range(args.steps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        step.replay()
        b.record()
        ts.append((a, b))
    b0.record()
    torch.cuda.synchronize()
    total_ms = a0.elapsed_time(b0)
    per = [a.elapsed_time(b) for a, b in ts]
    ms = total_ms / args.steps
    gbs = step.active_bytes / (ms * 1e-3) / 1e9
    out = {"workload": f"Llama-2-7B decode step of linears, {args.layers} layers x (select + GEMM) x "
                       "{qkv N=12288, o, gate/up N=22016, down}, B=64, density 0.48, one hipGraph (configs[4])",
           "ms_per_step": round(ms, 4), "step_ms_median": round(statistics.median(per), 4),
           "GBps_active": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "steps": args.steps,
           "warmup": args.warmup, "resident_weight_gb": round(step.resident_weight_bytes / 1e9, 3),
           "active_gb_per_step": round(step.active_bytes / 1e9, 4),
           "launches_per_step": len(step.layers) * len(step.layers[0]) * 2,
           "floor_ms_at_8TBps": round(step.active_bytes / 8e12 * 1e3, 4),
           "parity": "indices bit-exact and outputs within tolerance on the first and last layers"}
    if not args.no_cpu:
        cpu_ms = cpu_layer_us * args.layers / 1e3
        out.update({"cpu_ms_per_step": round(cpu_ms, 1), "cpu_cores": len(os.sched_getaffinity(0)),
                    "cpu_sample": "layer 0's four select + GEMM on the oracle CPU path (exact-L1 top-k, torch CPU "
                                  "gather + fp32 matmul), one run after a warm-up each, times the layer count",
                    "gpu_speedup_over_cpu": round(cpu_ms / ms, 1)})
    del step
    torch.cuda.empty_cache()
    return out


def run_decode(args, dev):
    """`--workload decode`: the configs[4] measurement as its own JSON line."""
    d = measure_decode(args, dev)
    line = {
        "metric": METRIC, "value": d["GBps_active"], "unit": "GB/s", "n_gpus": 1, "steps": d["steps"],
        "warmup": d["warmup"], "ms_per_step": d["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: torch seed 1234 on device, W~N(0,0.02), X~N(0,1) (Laplace(0,0.05) for down)",
        "config": {"workload": d["workload"], "resident_weight_gb": d["resident_weight_gb"],
                   "active_gb_per_step": d["active_gb_per_step"], "launches_per_step": d["launches_per_step"]},
        "step_ms_median": d["step_ms_median"],
        "floor_ms_at_8TBps": d["floor_ms_at_8TBps"],
    }
    print(json.dumps(line), flush=True)


PERSTEP_FIXTURE = os.path.join(ROOT, "tests", "golden", "perstep_smaps.npz")


def measure_perstep(args, dev, batches=None):
    """Oracle-map replay (the reference's headline benchmark,
    scripts/bench_perstep_actual_kernel_speedup.py): for each batch size, every group-step's
    S-map of 7 projections x 32 layers (tests/golden/perstep_smaps.npz, from the reference's
    results/oracle/perstep_batch_sweep.json) gives 224 GEMMs with density 1 - S and
    floor(density * nblk) random active blocks (BPS:84-87), as bsa_mi355x.replay builds them.
    Each distinct (shape, density) is timed once (the reference's unique-case method,
    BPS:148-172) with this build's sparse kernel, its dense variant and hipBLASLt (torch.mm),
    every one rotated over >= 1 GiB of distinct active weight; a step's speedup is
    sum(dense) / sum(sparse) over its 224 GEMMs, averaged over the 55 group-steps of a batch
    size, next to the reference's A100X numbers for the same maps.  Returns (rows per batch size,
    active bytes and µs summed over the timed sparse cases)."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from bsa_mi355x import replay
    from oracle import bsg_oracle as orc

    fx = replay.load_maps(PERSTEP_FIXTURE)
    if batches is None:
        batches = [int(b) for b in (args.batches.split(",") if args.batches else fx["ref_batch"])]
    cases_by_b = replay.cases_for_batches(fx, batches)
    need = {}
    for cases in cases_by_b.values():
        for name, tenths in cases:
            k, n = replay.SHAPES[name]
            na = replay.active_count(tenths, replay.nblk_of(name))
            need[name] = max(need.get(name, 1), copies_for(na * 64 * n * 2))
    pools = {name: ShapePool(name, k, n, dev, need.get(name, 1), seed=SEED + i)
             for i, (name, (k, n)) in enumerate(replay.SHAPES.items())}
    log("perstep: weight pools " + ", ".join(f"{p.name} x{p.copies}" for p in pools.values()))
    rng = np.random.default_rng(SEED)
    reps = max(3, min(args.steps, 10))

    def timed(fns):
        return _graph_time(fns, reps)[0] / len(fns)

    results = []
    total_bytes = 0.0
    total_us = 0.0
    for bt in batches:
        sel = replay.batch_rows(fx, bt)
        maps = fx["smap_tenths"][sel]  # [steps, 7, 32] sparsity in tenths
        cases = cases_by_b[bt]
        x = {name: torch.randn(bt, p.k, generator=torch.Generator().manual_seed(bt), dtype=torch.float32)
             .to(torch.float16).to(dev) for name, p in pools.items()}
        y = {name: torch.empty(bt, p.n, dtype=torch.float16, device=dev) for name, p in pools.items()}
        dense_us, mm_us = {}, {}
        for name, p in pools.items():
            pl = bsa.resolve_plan(bt, p.n, p.nblk, p.nblk, dev, None, dense=True)
            nd = copies_for(p.packed_bytes)
            dense_us[name] = timed([(lambda i=i: bsa.gemm_packed(x[name], p.packed[i], p.n, None, y[name], plan=pl,
                                                                  workspace_prefix=f"ps_dense_{name}"))
                                    for i in range(nd)])
            mm_us[name] = timed([(lambda w=w: torch.mm(x[name], w, out=y[name])) for w in p.w_kn(nd)])
        sparse_us = {}
        for name, tenths in cases:
            p = pools[name]
            na = replay.active_count(tenths, p.nblk)
            idx = torch.from_numpy(replay.random_blocks(rng, p.nblk, na)).to(dev)
            pl = bsa.resolve_plan(bt, p.n, p.nblk, na, dev, None)
            nc = min(p.copies, copies_for(na * 64 * p.n * 2))
            fns = [(lambda i=i: bsa.gemm_packed(x[name], p.packed[i], p.n, idx, y[name], plan=pl,
                                                workspace_prefix=f"ps_{name}")) for i in range(nc)]
            fns[0]()
            torch.cuda.synchronize()
            if tenths in (1, 5, 9):  # spot parity on three densities per shape (every case: tests/test_gpu_replay.py)
                ref = orc.gemm_ref(x[name].float().cpu().numpy(), np.ascontiguousarray(p.w_kn_np.T),
                                   idx.cpu().numpy())
                if not orc.within_tolerance(y[name].float().cpu().numpy(), ref):
                    raise SystemExit(f"perstep B={bt} {name} density {tenths / 10}: output outside tolerance")
            us = timed(fns)
            sparse_us[(name, tenths)] = us
            total_bytes += na * 64 * p.n * 2
            total_us += us
        step_own, step_mm, sparse_steps = [], [], []
        dense_total = sparse_total = 0.0
        for m in maps:
            d_sum, s_sum = replay.step_sums(m, dense_us, sparse_us)
            m_sum, _ = replay.step_sums(m, mm_us, sparse_us)
            step_own.append(d_sum / s_sum)
            step_mm.append(m_sum / s_sum)
            sparse_steps.append(s_sum)
            dense_total += d_sum
            sparse_total += s_sum
        # Kernel replay throughput as scripts/analyze_perstep_kernel_replay_throughput.py:22-44 defines
        # it: batch tokens (B x group-steps) over the summed step kernel times (not end-to-end tokens/s)
        tokens = bt * len(sel)
        ref_dense_ms = float(np.sum(fx["ref_step_dense_ms"][sel]))
        ref_sparse_ms = float(np.sum(fx["ref_step_sparse_ms"][sel]))
        ref_i = list(fx["ref_batch"]).index(bt) if bt in list(fx["ref_batch"]) else None
        row = {"B": bt, "group_steps": int(len(sel)), "mean_sparsity": round(float(fx["mean_sparsity"][sel].mean()), 4),
               "unique_cases": len(cases),
               "speedup_vs_own_dense": round(float(np.mean(step_own)), 3),
               "speedup_vs_hipblaslt": round(float(np.mean(step_mm)), 3),
               "reference_a100x_speedup_vs_cublas": (round(float(fx["ref_batch_speedup"][ref_i]), 3)
                                                     if ref_i is not None else None),
               "dense_us": {k: round(v, 2) for k, v in dense_us.items()},
               "hipblaslt_us": {k: round(v, 2) for k, v in mm_us.items()},
               "sparse_us_step_mean": round(float(np.mean(sparse_steps)), 1),
               "replay_tokens_per_s": {"dense": round(tokens / (dense_total * 1e-6), 1),
                                       "sparse": round(tokens / (sparse_total * 1e-6), 1),
                                       "throughput_speedup": round(dense_total / sparse_total, 3)},
               "reference_a100x_replay_tokens_per_s": {"dense": round(tokens / (ref_dense_ms * 1e-3), 1),
                                                       "sparse": round(tokens / (ref_sparse_ms * 1e-3), 1),
                                                       "throughput_speedup": round(ref_dense_ms / ref_sparse_ms, 3)}}
        results.append(row)
        log(json.dumps(row))
    del pools
    torch.cuda.empty_cache()
    return results, total_bytes, total_us


def measure_step_graphs(args, dev, steps_per_batch=0):
    """Each group-step of the reference's maps (tests/golden/perstep_smaps.npz) as one captured
    graph of its 224 GEMMs (bsa_mi355x.replay.StepGraphs: 32 layers x q, k, v, o, gate, up,
    down, ~13 GB of per-layer weights), against the dense step graph of the same batch size;
    the step speedup is dense step time over sparse step time, beside the reference's A100X
    speedup for the same group-step.  Layers 0 and 31 of each batch size's first group-step are
    checked against the oracle before timing.  steps_per_batch 0: every group-step."""
    import numpy as np
    import torch

    from bsa_mi355x import replay
    from oracle import bsg_oracle as orc

    fx = replay.load_maps(PERSTEP_FIXTURE)
    t0 = time.perf_counter()
    sg = replay.StepGraphs(dev)
    log(f"step graphs: {sg.resident_weight_bytes / 1e9:.2f} GB of packed weights ({time.perf_counter() - t0:.1f} s)")
    reps = 5
    w_host = {}

    def graph_ms(g):
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b))
        return statistics.median(ts)

    rows = []
    for bt in [int(v) for v in fx["ref_batch"]]:
        sel = replay.batch_rows(fx, bt)
        if steps_per_batch:
            sel = sel[:steps_per_batch]
        sg.set_batch(bt)
        g = sg.capture(None)
        dense_ms = graph_ms(g)
        del g
        rng = np.random.default_rng(SEED + bt)
        sparse_ms, speed, ref_speed, active = [], [], [], []
        for i, r in enumerate(sel):
            lists = sg.step_lists(fx["smap_tenths"][r], rng)
            g = sg.capture(lists)
            if i == 0:
                for li in sorted({0, sg.n_layers - 1}):
                    for pi, shape in enumerate(replay.PROJ_SHAPE):
                        key = (li, pi)
                        if key not in w_host:
                            k, n = replay.SHAPES[shape]
                            w_host[key] = np.ascontiguousarray(
                                orc.tile_unpermute(sg.packed[li][pi].cpu().numpy(), n).reshape(-1, n)[:k].T)
                        x = sg.x[shape].cpu().numpy()
                        ref = orc.gemm_ref(x, w_host[key], lists[li][pi].cpu().numpy())
                        if not orc.within_tolerance(sg.y[li][pi].float().cpu().numpy(), ref):
                            raise SystemExit(f"step graph B={bt} layer {li} {replay.PROJ_SHAPE[pi]}#{pi}: "
                                             "output outside tolerance")
            ms = graph_ms(g)
            del g
            sparse_ms.append(ms)
            speed.append(dense_ms / ms)
            ref_speed.append(float(fx["ref_step_speedup"][r]))
            active.append(sg.active_bytes(lists))
        row = {"B": bt, "group_steps": len(sel), "mean_sparsity": round(float(fx["mean_sparsity"][sel].mean()), 4),
               "dense_step_ms": round(dense_ms, 4), "sparse_step_ms_mean": round(float(np.mean(sparse_ms)), 4),
               "speedup_vs_own_dense": round(float(np.mean(speed)), 3),
               "reference_a100x_step_speedup_same_steps": round(float(np.mean(ref_speed)), 3),
               "sparse_GBps_active": round(float(np.mean(active)) / (float(np.mean(sparse_ms)) * 1e-3) / 1e9, 1),
               "dense_GBps": round(sg.active_bytes(None) / (dense_ms * 1e-3) / 1e9, 1),
               "tokens_per_s_sparse": round(bt / (float(np.mean(sparse_ms)) * 1e-3), 1)}
        rows.append(row)
        log(f"step graph B={bt}: {json.dumps(row)}")
    del sg
    torch.cuda.empty_cache()
    return rows


def run_perstep(args, dev):
    """`--workload perstep`: the reference's headline table (every batch size) as one JSON line."""
    results, total_bytes, total_us = measure_perstep(args, dev)
    graphs = measure_step_graphs(args, dev)
    batches = [r["B"] for r in results]
    reps = max(3, min(args.steps, 10))
    line = {
        "metric": METRIC, "value": round(total_bytes / (total_us * 1e-6) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": reps, "warmup": 2, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "reference S-maps (results/oracle/perstep_batch_sweep.json via tests/golden/perstep_smaps.npz); "
                "W~N(0,0.02), X~N(0,1) synthetic; random masks floor(density*nblk); each case rotates over >=1 GiB "
                "of distinct active weight",
        "config": {"workload": "oracle-map replay of the 224-GEMM decode step (7 projections x 32 layers), "
                               "B in " + ",".join(map(str, batches)) + " (the reference's headline speedup table)",
                   "value_is": "active-weight bytes / time over every distinct timed sparse case"},
        "perstep": results,
        "step_graphs": graphs,
    }
    print(json.dumps(line), flush=True)


def _pct(v, q):
    v = sorted(v)
    return v[min(len(v) - 1, max(0, int(round(q * (len(v) - 1)))))]


def run_timeline(args, dev):
    """Per-work-group phase timeline of one point (--only NAME of the llama workload), with the
    profiling build of the library (libbsgemm_timeline.so: the same kernels, each work-group's wave
    0 stamping the 100 MHz wall clock at its phase boundaries).  The point's R rotated launches are
    captured as one graph (the bench's rotation) and replayed; the stamps of the last replay give,
    per launch, each work-group's phases relative to the launch's first work-group start:
    dispatch skew, list staging, first block consumed, main loop (wave 0), how long after wave 0
    the work-group's last wave ended its loop (last_wave_lag, inside the epilogue), epilogue,
    hand-off/end.  Also
    reports the per-launch time of the graph, whose excess over the stamped span is the gap
    between kernels."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa

    lib = bsa.load()
    if not args.only:
        raise SystemExit("--workload timeline needs --only POINT")
    khz = int(lib.bsg_timeline_clock_khz())
    rows = [r for r in matrix_points("llama", dev) if r[0] == args.only]
    if not rows:
        raise SystemExit(f"--only {args.only}: no such point")
    name, sh, bt, na, dense = rows[0]
    pool = ShapePool(sh, *SHAPES[sh], dev, copies_for(na * 64 * SHAPES[sh][1] * 2))
    plan = bsa.Plan(*[int(v) for v in args.plan.split(",")]) if args.plan else None
    pt = Point(name, pool, bt, na, dev, dense=dense, plan=plan)
    rf, ok = pt.check()
    if not ok:
        raise SystemExit(f"{name}: parity failure (rel_fro {rf})")
    if args.select:
        from bsa_mi355x.select import select_gemm_packed

        sel_idx = torch.empty(na, dtype=torch.int32, device=dev)
        sel_cnt = torch.empty(1, dtype=torch.int32, device=dev)

        def launch_select(i):
            select_gemm_packed(pt.x, pool.packed[i % pt.copies], pt.n, na, pt.y, plan=pt.plan, idx_out=sel_idx,
                               count_out=sel_cnt, workspace_prefix="tl_select")

        pt.launch = launch_select
    groups = 1 << 16
    buf = torch.zeros(pt.copies * groups * 8, dtype=torch.int64, device=dev)
    rc = lib.bsg_timeline_attach(buf.data_ptr(), pt.copies, groups)
    if rc != 0:
        raise SystemExit("the timeline workload needs BSA_MI355X_LIB=timeline (the profiling build): "
                         + lib.bsg_last_error().decode())
    pt.capture()
    lib.bsg_timeline_attach(None, 0, 0)
    reps = max(5, args.steps)
    for _ in range(2):
        pt.graph.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        pt.graph.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1000.0 / pt.copies)
    per_launch = statistics.median(ts)
    st = buf.view(pt.copies, groups, 8).cpu().numpy()
    us = 1e3 / khz
    phases = {"dispatch_skew": [], "list_staging": [], "first_block": [], "main_loop": [], "last_wave_lag": [],
              "epilogue": [], "handoff_end": [], "end_offset": []}
    last = {"handoff_end": [], "end_offset": []}
    spans, end_spread = [], []
    n_groups = 0
    for li in range(pt.copies):
        g = st[li]
        live = g[:, 5] > 0
        g = g[live]
        if len(g) == 0:
            continue
        n_groups = len(g)
        t0 = g[:, 0].min()
        spans.append((g[:, 5].max() - t0) * us)
        end_spread.append((g[:, 5].max() - np.median(g[:, 5])) * us)
        phases["dispatch_skew"] += list((g[:, 0] - t0) * us)
        phases["list_staging"] += list((g[:, 1] - g[:, 0]) * us)
        first = np.where(g[:, 2] > 0, g[:, 2], g[:, 3])
        phases["first_block"] += list((first - g[:, 1]) * us)
        phases["main_loop"] += list((g[:, 3] - first) * us)
        last_end = g[:, 6] >> 1  # the work-group's last wave to end its main loop
        phases["last_wave_lag"] += list((np.maximum(last_end, g[:, 3]) - g[:, 3]) * us)
        phases["epilogue"] += list((g[:, 4] - g[:, 3]) * us)
        phases["handoff_end"] += list((g[:, 5] - g[:, 4]) * us)
        phases["end_offset"] += list((g[:, 5] - t0) * us)
        ly = (g[:, 6] & 1) == 1
        last["handoff_end"] += list((g[ly, 5] - g[ly, 4]) * us)
        last["end_offset"] += list((g[ly, 5] - t0) * us)
    summary = {k: {"median": round(float(np.median(v)), 3), "p10": round(float(_pct(v, 0.1)), 3),
                   "p90": round(float(_pct(v, 0.9)), 3)} for k, v in phases.items() if v}
    summary_last = {k: {"median": round(float(np.median(v)), 3), "p90": round(float(_pct(v, 0.9)), 3)}
                    for k, v in last.items() if v}
    xcc = st[0, : n_groups, 7] >> 32
    line = {"workload": "timeline", "point": name, "B": bt, "K": pt.k, "N": pt.n, "active_blocks": pt.na,
            "plan": list(pt.plan.as_tuple()), "kernel": KERNEL_NAMES.get(pt.plan.kind), "launches": pt.copies,
            "work_groups": int(n_groups), "clock_khz": khz,
            "us_per_launch_graph": round(per_launch, 3),
            "stamped_span_us": {"median": round(float(np.median(spans)), 3), "p90": round(float(_pct(spans, 0.9)), 3)},
            "gap_between_kernels_us": round(per_launch - float(np.median(spans)), 3),
            "end_spread_us": round(float(np.median(end_spread)), 3),
            "phases_us": summary, "y_storing_groups_us": summary_last,
            "groups_per_xcc": np.bincount(xcc.astype(np.int64), minlength=8).tolist()}
    print(json.dumps(line), flush=True)


def main():
    args = parse_args()
    if args.workload == "timeline":
        # select the profiling build before the library is first loaded
        os.environ["BSA_MI355X_LIB"] = "timeline"
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} requested); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import bsa_mi355x as bsa

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration, args.steps)
        return
    bsa.load()
    log(f"device {torch.cuda.get_device_name(dev)}; lib {bsa.load().bsg_version().decode()}")
    if args.workload in ("llama", "down_sweep"):
        run_matrix(args, dev)
    elif args.workload == "fused":
        run_fused(args, dev)
    elif args.workload == "rule":
        print(json.dumps({"metric": METRIC, "rule_select_gemm": measure_rule_linear(args, dev)}), flush=True)
    elif args.workload == "perstep":
        run_perstep(args, dev)
    elif args.workload == "2d":
        run_2d(args, dev)
    elif args.workload == "timeline":
        run_timeline(args, dev)
    else:
        run_decode(args, dev)


if __name__ == "__main__":
    main()
