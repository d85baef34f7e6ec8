#!/usr/bin/env python3
"""Benchmark of the MI355X batch-shared block-sparse GEMM (one JSON line on stdout).

Workload: Llama-2-7B down_proj, B=16, K=11008 (172 blocks of 64),
N=4096, fp16, sweeping block sparsity {0, 0.25, 0.5, 0.638, 0.8}; the 0% point runs the same
kernel with every block active (the in-run dense baseline).  One "step" = one replay of a
hipGraph holding every sweep point's R back-to-back GEMM launches, each on a different copy of
the packed weight (R copies span >= 1 GiB, so the 256 MB Infinity Cache cannot serve a repeat
and the bytes really come from HBM).  Per-point µs/GEMM come from each point's own graph.

value  = active-weight bytes of all GEMMs in the timed steps / timed seconds (GB/s)
roofline = the s=0.5 sparse GEMM (86/172 blocks): algorithmic bytes na*64*N*2 per launch over
           the average launch duration from HIP events around its graph replays.
cpu_baseline = the oracle's CPU path (torch CPU gather + fp32 matmul) on the s=0.5 point.

    python bench.py [--steps K] [--warmup W] [--workload down_sweep|llama|fused|decode|perstep]
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
METRIC = "µs/GEMM + HBM GB/s + speedup vs dense, Llama-2-7B shapes at B=2/16/64"
# Committed PMC summaries (HBM bytes per launch) of the roofline point of each workload.
TRAFFIC_PROFILES = {
    "down_b16_s500": os.path.join(ROOT, "profiles", "traffic_bsg_gemm_down_b16_s500.md"),
    "gate_up_b64_s520": os.path.join(ROOT, "profiles", "traffic_bsg_gemm_xl_gate_up_b64_s520.md"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="down_sweep",
                    choices=["down_sweep", "llama", "fused", "decode", "perstep", "2d"])
    ap.add_argument("--batches", default=None, help="perstep workload: batch sizes (default: all six)")
    ap.add_argument("--layers", type=int, default=32, help="decode workload: number of layers")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, help="time only this point (profiling runs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the GEMMs, replay a plain device copy of MIB MiB (PMC calibration)")
    return ap.parse_args()


class Point:
    """One GEMM configuration: packed weight copies + a graph of R rotated launches."""

    def __init__(self, name, bt, k, n, na, x_dist, seed, dev, dense=False, plan=None):
        import numpy as np
        import torch

        import bsa_mi355x as bsa
        from oracle import bsg_oracle as orc

        self.name, self.bt, self.k, self.n, self.na, self.dense = name, bt, k, n, na, dense
        nb = orc.nblk_of(k)
        self.nblk = nb
        x, w_kn, idx = orc.make_inputs(seed, bt, k, n, x_dist, na=(nb if dense else na))
        self.x_np, self.w_kn_np, self.idx_np = x, w_kn, idx
        self.x = torch.from_numpy(x).to(dev)
        w_kn_t = torch.from_numpy(w_kn).to(dev)
        packed = bsa.pack_weight(w_kn_t, layout="kn")
        del w_kn_t
        self.copies = max(1, math.ceil(ROTATE_BYTES / packed.numel() / 2))
        self.packed = [packed] + [packed.clone() for _ in range(self.copies - 1)]
        self.idx = torch.from_numpy(idx).to(dev)
        self.y = torch.empty(bt, n, dtype=torch.float16, device=dev)
        self.plan = bsa.resolve_plan(bt, n, nb, nb if dense else na, dev, plan, dense=dense)
        self.active_bytes = (nb if dense else na) * 64 * n * 2
        self.flops = 2 * bt * (nb if dense else na) * 64 * n
        self.graph = None

    def launch(self, i):
        import bsa_mi355x as bsa

        p = self.packed[i % self.copies]
        if self.dense:
            bsa.gemm_packed(self.x, p, self.n, None, self.y, plan=self.plan, workspace_prefix=f"bench_{self.name}")
        else:
            bsa.gemm_packed(self.x, p, self.n, self.idx, self.y, plan=self.plan, workspace_prefix=f"bench_{self.name}")

    def capture(self):
        import torch

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(self.copies):
                self.launch(i)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(self.copies):
                self.launch(i)
        torch.cuda.synchronize()
        self.graph = g

    def check(self):
        """Parity of the benchmarked launch against the oracle (fp32 CPU path)."""
        import numpy as np
        import torch

        from oracle import bsg_oracle as orc

        self.launch(0)
        torch.cuda.synchronize()
        w_nk = np.ascontiguousarray(self.w_kn_np.T)
        ref = orc.gemm_ref(self.x_np, w_nk, self.idx_np)
        y = self.y.float().cpu().numpy()
        return orc.rel_frobenius(y, ref), orc.within_tolerance(y, ref)


def capture_step(points):
    """One hipGraph holding a whole step: every point's R rotated launches, back to back."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for p in points:
            for i in range(p.copies):
                p.launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for p in points:
            for i in range(p.copies):
                p.launch(i)
    torch.cuda.synchronize()
    return g


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


def cpu_baseline(point, seconds):
    import torch

    from oracle import bsg_oracle as orc

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x = torch.from_numpy(point.x_np)
    w = torch.from_numpy(point.w_kn_np)
    idx = torch.from_numpy(point.idx_np.astype("int64"))
    for _ in range(2):
        orc.gemm_ref_torch(x, w, idx)
    samples = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(samples) < 500:
        t = time.perf_counter_ns()
        orc.gemm_ref_torch(x, w, idx)
        samples.append((time.perf_counter_ns() - t) / 1e3)
    us = statistics.median(samples)
    return {
        "value": round(point.active_bytes / (us * 1e-6) / 1e9, 2),
        "unit": "GB/s",
        "us_per_gemm": round(us, 1),
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle gemm_ref_torch (torch CPU gather + fp32 matmul) on {point.name}: B={point.bt} "
                   f"K={point.k} N={point.n} {point.na}/{point.nblk} blocks; {len(samples)} timed runs after 2 "
                   f"warm-ups, median"),
    }


def cpu_point_us(point, runs=5):
    """The same op on the oracle's CPU path (torch CPU gather + fp32 matmul, every host core): the
    median of a few runs after one warm-up, shown beside each point's GPU time."""
    import torch

    from oracle import bsg_oracle as orc

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    x = torch.from_numpy(point.x_np)
    w = torch.from_numpy(point.w_kn_np)
    idx = torch.from_numpy(point.idx_np.astype("int64"))
    orc.gemm_ref_torch(x, w, idx)
    samples = []
    for _ in range(runs):
        t = time.perf_counter_ns()
        orc.gemm_ref_torch(x, w, idx)
        samples.append((time.perf_counter_ns() - t) / 1e3)
    return statistics.median(samples)


def load_traffic(point):
    """HBM bytes per launch of a roofline point, from its committed PMC summary (a line
    `traffic_bytes_per_launch: <int>`), or None when that point has no summary."""
    path = TRAFFIC_PROFILES.get(point)
    if path is None:
        return None
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


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
    """hipBLASLt dense GEMM (torch.mm) on the same shape, rotated over weight copies: context."""
    import torch

    w0 = torch.from_numpy(point.w_kn_np).to(point.x.device)
    ws = [w0] + [w0.clone() for _ in range(point.copies - 1)]
    out = torch.empty(point.bt, point.n, dtype=torch.float16, device=point.x.device)
    torch.mm(point.x, ws[0], out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for w in ws:
            torch.mm(point.x, w, out=out)
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
        ts.append(a.elapsed_time(b) * 1000.0 / len(ws))
    del g, ws
    return statistics.median(ts)


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
            rc = lib.bsg_read_calibrate(point.packed[i].data_ptr(), nbytes, sink.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(lib.bsg_last_error().decode())
        return f

    med, _ = _graph_time([launch(i) for i in range(point.copies)], reps)
    return med / point.copies


KERNEL_NAMES = {1: "bsg_gemm_kernel", 2: "bsg_gemm_xl_kernel", 3: "bsg_gemm_fma_kernel"}


def _graph_time(fns, reps, warmup=2):
    """Capture fns back to back as one graph; median µs per replay over `reps` replays."""
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
    return statistics.median(ts), statistics.mean(ts)


def run_2d(args, dev):
    """2-D block sparsity (active output blocks as well as K-blocks): down_proj B=16 with half of the K-blocks
    active and a sweep of active 64-column output blocks, in place and compact.  Each point is
    a graph of launches rotated over >= 1 GiB of weight copies; parity against the oracle
    first.  Bytes per launch: na * 64 * (nn * 64) * 2 (active weight)."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from bsa_mi355x import sparse2d
    from oracle import bsg_oracle as orc

    bt, k, n = 16, 11008, 4096
    nb_k, nb_n = orc.nblk_of(k), n // 64
    x, w_kn, kidx = orc.make_inputs(1234, bt, k, n, "laplace", na=orc.n_active_for_sparsity(0.5, nb_k))
    rng = np.random.default_rng(4321)
    xt, kt = torch.from_numpy(x).to(dev), torch.from_numpy(kidx).to(dev)
    packed0 = bsa.pack_weight(torch.from_numpy(w_kn).to(dev), layout="kn")
    copies = max(1, math.ceil(ROTATE_BYTES / packed0.numel() / 2))
    packed = [packed0] + [packed0.clone() for _ in range(copies - 1)]
    w_nk = np.ascontiguousarray(w_kn.T)
    reps = max(5, args.steps)
    rows, total_bytes, total_us, focus = [], 0, 0.0, None
    for nd, compact in ((1.0, False), (0.75, False), (0.5, False), (0.25, False), (0.5, True)):
        nn = int(round(nd * nb_n))
        nidx = np.sort(rng.choice(nb_n, nn, replace=False)).astype(np.int32)
        nt = torch.from_numpy(nidx).to(dev)
        y = torch.zeros(bt, nn * 64 if compact else n, dtype=torch.float16, device=dev)
        pl = sparse2d.plan_2d(bt, n, nn, nb_k, len(kidx), dev)

        def call(i, nt=nt, y=y, compact=compact, pl=pl):
            return lambda: sparse2d.gemm_2d_packed(xt, packed[i % copies], n, kt, nt, y, compact=compact, plan=pl,
                                                   workspace_prefix="bench2d")

        call(0)()
        torch.cuda.synchronize()
        want = orc.gemm_2d_ref(x, w_nk, kidx, nidx, out_init=np.zeros((bt, n), np.float32), compact=compact)
        if not orc.within_tolerance(y.float().cpu().numpy(), want):
            raise SystemExit(f"2-D parity failure at n-density {nd} compact={compact}")
        med, mean = _graph_time([call(i) for i in range(copies)], reps)
        us, us_mean = med / copies, mean / copies
        b = len(kidx) * 64 * nn * 64 * 2
        total_bytes += b * copies
        total_us += med
        name = f"down_b16_k500_n{int(round(nd * 1000)):04d}{'_compact' if compact else ''}"
        row = {"name": name, "active_k_blocks": len(kidx), "active_n_blocks": nn, "compact": compact,
               "us_per_gemm": round(us, 3), "GBps_active": round(b / (us * 1e-6) / 1e9, 1), "plan": list(pl.as_tuple())}
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
                "output-block masks rng.choice seed 4321; weights rotated over >=1 GiB of copies",
        "config": {"workload": "2-D block sparsity: down_proj B=16 K=11008 N=4096, K density 0.5, output-block "
                               "density {1, 0.75, 0.5, 0.25} in place + 0.5 compact"},
        "points": rows,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "bsg_gemm_kernel (2-D)",
                     "point": frow["name"], "avg_launch_us": round(fmean, 3), "bytes_per_launch": fb},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def run_fused(args, dev):
    """fused exact-L1 selection (k=31 of 64) + sparse GEMM on gate/up at B=64
    (K=4096 -> N=11008), rotated over >= 1 GiB of weight copies; indices checked bit-exact."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from bsa_mi355x.select import select_gemm_packed
    from oracle import bsg_oracle as orc

    bt, k, n, keep = 64, 4096, 11008, 31
    pt = Point("gate_up_b64_fused", bt, k, n, keep, "normal", 1234, dev)
    idx = torch.empty(keep, dtype=torch.int32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    select_gemm_packed(pt.x, pt.packed[0], n, keep, pt.y, idx_out=idx, count_out=cnt, workspace_prefix="fused_bench")
    torch.cuda.synchronize()
    want = orc.select_topk_l1(pt.x_np, keep)
    got = idx.cpu().numpy()
    if not np.array_equal(got, want) or int(cnt.item()) != keep:
        raise SystemExit(f"fused selector indices differ from the oracle: {got} vs {want}")
    y_ref = orc.gemm_ref(pt.x_np, np.ascontiguousarray(pt.w_kn_np.T), want)
    if not orc.within_tolerance(pt.y.float().cpu().numpy(), y_ref):
        raise SystemExit("fused select+GEMM output outside tolerance")
    log("fused: indices bit-exact, GEMM within tolerance")
    plan = bsa.resolve_plan(bt, n, pt.nblk, keep, dev)
    ws_sel = "fused_sel"

    def fused(i):
        return lambda: select_gemm_packed(pt.x, pt.packed[i], n, keep, pt.y, plan=plan, idx_out=idx, count_out=cnt,
                                          workspace_prefix="fused_bench")

    def gemm_only(i):
        return lambda: bsa.gemm_packed(pt.x, pt.packed[i], n, idx, pt.y, plan=plan, workspace_prefix="fused_gemm")

    def select_only(i):
        return lambda: bsa.select_topk_l1(pt.x, keep, idx_out=idx, count_out=cnt, workspace_prefix=ws_sel)

    r = pt.copies
    reps = max(5, args.steps)
    t_fused = _graph_time([fused(i) for i in range(r)], reps)[0] / r
    t_gemm = _graph_time([gemm_only(i) for i in range(r)], reps)[0] / r
    t_sel = _graph_time([select_only(i) for i in range(r)], reps)[0] / r
    gbs = pt.active_bytes / (t_fused * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": reps,
        "warmup": 2, "ms_per_step": round(t_fused * r / 1000.0, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: numpy PCG64 seed 1234, W~N(0,0.02) [K,N], X~N(0,1); weights rotated over >=1 GiB",
        "config": {"workload": "fused exact-L1 select (k=31 of 64) + sparse GEMM, gate/up B=64 K=4096 N=11008 "
                               "(configs[3])", "plan": list(plan.as_tuple())},
        "us_select_plus_gemm": round(t_fused, 3), "us_gemm_only": round(t_gemm, 3), "us_select_only": round(t_sel, 3),
        "indices_bit_exact": True,
    }
    print(json.dumps(line), flush=True)


def run_decode(args, dev):
    """Llama-2-7B-shaped decode step of linears (layers x {qkv, o, gate/up,
    down}), B=64, per-projection masks from the fused selector at density 0.48 (k=31/64, 83/172),
    the whole step captured as one hipGraph."""
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
    # parity: first and last layer, every projection (indices bit-exact, outputs within tolerance)
    for li in sorted({0, args.layers - 1}):
        for p in step.layers[li]:
            x = p.x.cpu().numpy()
            want = orc.select_topk_l1(x, p.keep)
            got = p.idx[: min(p.keep, p.nblk)].cpu().numpy()
            if not np.array_equal(got, want):
                raise SystemExit(f"decode layer {li} {p.name}: selected blocks differ from the oracle")
            w_nk = orc.tile_unpermute(p.packed.cpu().numpy(), p.n).reshape(-1, p.n)[: p.k].T
            if not orc.within_tolerance(p.y.float().cpu().numpy(), orc.gemm_ref(x, np.ascontiguousarray(w_nk), want)):
                raise SystemExit(f"decode layer {li} {p.name}: output outside tolerance")
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
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: torch seed 1234 on device, W~N(0,0.02), X~N(0,1) (Laplace(0,0.05) for down)",
        "config": {"workload": f"Llama-2-7B decode step of linears, {args.layers} layers x (select + GEMM) x "
                               "{qkv N=12288, o, gate/up N=22016, down}, B=64, density 0.48, one hipGraph (configs[4])",
                   "resident_weight_gb": round(step.resident_weight_bytes / 1e9, 3),
                   "active_gb_per_step": round(step.active_bytes / 1e9, 4),
                   "launches_per_step": 8 * args.layers},
        "step_ms_median": round(statistics.median(per), 4),
        "floor_ms_at_8TBps": round(step.active_bytes / 8e12 * 1e3, 4),
    }
    print(json.dumps(line), flush=True)


PERSTEP_FIXTURE = os.path.join(ROOT, "tests", "golden", "perstep_smaps.npz")
PERSTEP_SHAPES = {"qkvo": (4096, 4096), "gate_up": (4096, 11008), "down": (11008, 4096)}
PERSTEP_PROJ_SHAPE = ["qkvo", "qkvo", "qkvo", "qkvo", "gate_up", "gate_up", "down"]


class ShapePool:
    """Packed-weight copies (>= 1 GiB) of one projection shape, plus [K,N] copies for
    torch.mm, shared by every density and batch of the per-step replay."""

    def __init__(self, name, k, n, dev, seed):
        import numpy as np
        import torch

        import bsa_mi355x as bsa

        self.name, self.k, self.n = name, k, n
        self.nblk = (k + 63) // 64
        rng = np.random.default_rng(seed)
        w_kn = (rng.standard_normal((k, n), dtype=np.float32) * 0.02).astype(np.float16)
        self.w_kn_np = w_kn
        w0 = torch.from_numpy(w_kn).to(dev)
        p0 = bsa.pack_weight(w0, layout="kn")
        self.copies = max(1, math.ceil(ROTATE_BYTES / (p0.numel() * 2)))
        self.packed = [p0] + [p0.clone() for _ in range(self.copies - 1)]
        self.w_kn = [w0] + [w0.clone() for _ in range(self.copies - 1)]


def run_perstep(args, dev):
    """Oracle-map replay (the reference's headline benchmark,
    scripts/bench_perstep_actual_kernel_speedup.py): for each batch size, every group-step's
    S-map of 7 projections x 32 layers (tests/golden/perstep_smaps.npz, from the reference's
    results/oracle/perstep_batch_sweep.json) gives 224 GEMMs with density 1 - S and
    floor(density * nblk) random active blocks (BPS:84-87).  Each distinct (shape, density) is
    timed once (the reference's unique-case method, BPS:148-172) with this build's sparse kernel,
    its dense variant and hipBLASLt (torch.mm), every one rotated over >= 1 GiB of weight
    copies; a step's speedup is sum(dense) / sum(sparse) over its 224 GEMMs, averaged over the
    55 group-steps of a batch size, next to the reference's A100X numbers for the same maps."""
    import numpy as np
    import torch

    import bsa_mi355x as bsa
    from oracle import bsg_oracle as orc

    fx = np.load(PERSTEP_FIXTURE, allow_pickle=False)
    batches = [int(b) for b in (args.batches.split(",") if args.batches else fx["ref_batch"])]
    pools = {name: ShapePool(name, k, n, dev, 1234 + i) for i, (name, (k, n)) in enumerate(PERSTEP_SHAPES.items())}
    log("perstep: weight pools " + ", ".join(f"{p.name} x{p.copies}" for p in pools.values()))
    rng = np.random.default_rng(1234)
    reps = max(3, min(args.steps, 10))

    def timed(fns):
        return _graph_time(fns, reps)[0] / len(fns)

    results = []
    total_bytes = 0.0
    total_us = 0.0
    for bt in batches:
        sel = np.nonzero(fx["batch"] == bt)[0]
        maps = fx["smap_tenths"][sel]  # [steps, 7, 32] sparsity in tenths
        cases = sorted({(PERSTEP_PROJ_SHAPE[pi], 10 - int(t)) for m in maps for pi in range(7) for t in m[pi]})
        x = {name: torch.randn(bt, p.k, generator=torch.Generator().manual_seed(bt), dtype=torch.float32)
             .to(torch.float16).to(dev) for name, p in pools.items()}
        y = {name: torch.empty(bt, p.n, dtype=torch.float16, device=dev) for name, p in pools.items()}
        dense_us, mm_us = {}, {}
        for name, p in pools.items():
            pl = bsa.resolve_plan(bt, p.n, p.nblk, p.nblk, dev, None, dense=True)
            dense_us[name] = timed([(lambda i=i: bsa.gemm_packed(x[name], p.packed[i], p.n, None, y[name], plan=pl,
                                                                  workspace_prefix=f"ps_dense_{name}"))
                                    for i in range(p.copies)])
            mm_us[name] = timed([(lambda i=i: torch.mm(x[name], p.w_kn[i], out=y[name])) for i in range(p.copies)])
        sparse_us = {}
        for name, tenths in cases:
            p = pools[name]
            na = max(1, min(p.nblk, int(math.floor(tenths / 10.0 * p.nblk))))
            idx = torch.from_numpy(np.sort(rng.choice(p.nblk, na, replace=False)).astype(np.int32)).to(dev)
            pl = bsa.resolve_plan(bt, p.n, p.nblk, na, dev, None)
            fns = [(lambda i=i: bsa.gemm_packed(x[name], p.packed[i], p.n, idx, y[name], plan=pl,
                                                workspace_prefix=f"ps_{name}")) for i in range(p.copies)]
            fns[0]()
            torch.cuda.synchronize()
            if tenths in (1, 5, 9):  # spot parity on three densities per shape
                ref = orc.gemm_ref(x[name].float().cpu().numpy(), np.ascontiguousarray(p.w_kn_np.T),
                                   idx.cpu().numpy())
                if not orc.within_tolerance(y[name].float().cpu().numpy(), ref):
                    raise SystemExit(f"perstep B={bt} {name} density {tenths / 10}: output outside tolerance")
            us = timed(fns)
            sparse_us[(name, tenths)] = (us, na)
            total_bytes += na * 64 * p.n * 2
            total_us += us
        step_own, step_mm = [], []
        dense_total = sparse_total = 0.0
        for m in maps:
            d_sum = m_sum = s_sum = 0.0
            for pi in range(7):
                name = PERSTEP_PROJ_SHAPE[pi]
                for t in m[pi]:
                    us, _ = sparse_us[(name, 10 - int(t))]
                    s_sum += us
                    d_sum += dense_us[name]
                    m_sum += mm_us[name]
            step_own.append(d_sum / s_sum)
            step_mm.append(m_sum / s_sum)
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
               "sparse_us_step_mean": round(float(np.mean([sum(sparse_us[(PERSTEP_PROJ_SHAPE[pi], 10 - int(t))][0]
                                                               for pi in range(7) for t in m[pi]) for m in maps])), 1),
               "replay_tokens_per_s": {"dense": round(tokens / (dense_total * 1e-6), 1),
                                       "sparse": round(tokens / (sparse_total * 1e-6), 1),
                                       "throughput_speedup": round(dense_total / sparse_total, 3)},
               "reference_a100x_replay_tokens_per_s": {"dense": round(tokens / (ref_dense_ms * 1e-3), 1),
                                                       "sparse": round(tokens / (ref_sparse_ms * 1e-3), 1),
                                                       "throughput_speedup": round(ref_dense_ms / ref_sparse_ms, 3)}}
        results.append(row)
        log(json.dumps(row))
    line = {
        "metric": METRIC, "value": round(total_bytes / (total_us * 1e-6) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": reps, "warmup": 2, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "reference S-maps (results/oracle/perstep_batch_sweep.json via tests/golden/perstep_smaps.npz); "
                "W~N(0,0.02), X~N(0,1) synthetic; random masks floor(density*nblk); weights rotated over >=1 GiB",
        "config": {"workload": "oracle-map replay of the 224-GEMM decode step (7 projections x 32 layers), "
                               "B in " + ",".join(map(str, batches)) + " (the reference's headline speedup table)",
                   "value_is": "active-weight bytes / time over every distinct timed sparse case"},
        "perstep": results,
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} requested); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import bsa_mi355x as bsa
    from oracle import bsg_oracle as orc

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration, args.steps)
        return
    bsa.load()
    log(f"device {torch.cuda.get_device_name(dev)}; lib {bsa.load().bsg_version().decode()}")

    if args.workload == "down_sweep":
        k, n, bt = 11008, 4096, 16
        points = []
        for s in (0.0, 0.25, 0.5, 0.638, 0.8):
            na = orc.n_active_for_sparsity(s, orc.nblk_of(k))
            name = "down_b16_dense" if s == 0.0 else f"down_b16_s{int(round(s * 1000)):03d}"
            points.append(Point(name, bt, k, n, na, "laplace", 1234, dev, dense=(s == 0.0)))
            log(f"prepared {name}: na={na} copies={points[-1].copies} plan={points[-1].plan}")
        workload = "down_proj B=16 K=11008 N=4096 fp16, block sparsity sweep {0,0.25,0.5,0.638,0.8} (configs[1])"
        focus = "down_b16_s500"
    elif args.workload == "llama":
        shapes = {"qkvo": (4096, 4096), "gate_up": (4096, 11008), "down": (11008, 4096)}
        points = []
        for bt, s in ((2, 0.803), (16, 0.638), (64, 0.520)):
            for sh, (k, n) in shapes.items():
                na = orc.n_active_for_sparsity(s, orc.nblk_of(k))
                name = f"{sh}_b{bt}_s{int(round(s * 1000)):03d}"
                points.append(Point(name, bt, k, n, na, "laplace" if sh == "down" else "normal", 1234, dev))
                points.append(Point(f"{sh}_b{bt}_dense", bt, k, n, na, "laplace" if sh == "down" else "normal", 1234,
                                    dev, dense=True))
                log(f"prepared {name}: na={na} plan={points[-2].plan}")
        workload = "Llama-2-7B q/k/v/o, gate/up, down at B=2@0.803, B=16@0.638, B=64@0.520 (configs[2])"
        focus = "gate_up_b64_s520"
    elif args.workload == "fused":
        run_fused(args, dev)
        return
    elif args.workload == "perstep":
        run_perstep(args, dev)
        return
    elif args.workload == "2d":
        run_2d(args, dev)
        return
    else:
        run_decode(args, dev)
        return

    if args.only:
        points = [p for p in points if p.name == args.only]
        if not points:
            raise SystemExit(f"--only {args.only}: no such point")
        focus = points[0].name
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
    step_graph = capture_step(points)
    log("graphs captured")

    total_ms, wall, per = time_points(points, step_graph, args.steps, args.warmup)
    step_bytes = sum(p.active_bytes * p.copies for p in points)
    value = step_bytes * args.steps / (total_ms * 1e-3) / 1e9
    log(f"timed {args.steps} steps in {total_ms:.2f} ms (host wall {wall * 1e3:.1f} ms)")

    dense_us = {}
    for p in points:
        if p.dense:
            dense_us[p.name.replace("_dense", "")] = per[p.name][0]
    out_points = []
    for p in points:
        med, mean = per[p.name]
        gbs = p.active_bytes / (med * 1e-6) / 1e9
        row = {"name": p.name, "B": p.bt, "K": p.k, "N": p.n, "active_blocks": p.nblk if p.dense else p.na,
               "nblk": p.nblk, "us_per_gemm": round(med, 3), "GBps_active": round(gbs, 1),
               "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
               "plan": list(p.plan.as_tuple())}
        if p.bt >= 16:
            row["mfma_util"] = round(p.flops / (med * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 5)
        if not p.dense:
            key = p.name.rsplit("_s", 1)[0] if args.workload == "llama" else "down_b16"
            d = dense_us.get(key)
            if d:
                row["speedup_vs_dense"] = round(d / med, 3)
                row["ideal_speedup"] = round(p.nblk / p.na, 3)
                row["speedup_over_ideal"] = round((d / med) / (p.nblk / p.na), 3)
        out_points.append(row)
        log(json.dumps(row))

    fp = next(p for p in points if p.name == focus)
    f_med, f_mean = per[focus]
    achieved = fp.active_bytes / (f_mean * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic(focus),
                "kernel": KERNEL_NAMES.get(fp.plan.kind, "bsg_gemm"), "point": focus,
                "avg_launch_us": round(f_mean, 3), "bytes_per_launch": fp.active_bytes}
    if not args.only:
        rd = read_calibration_us(fp)
        roofline["practical_read"] = {
            "us_per_launch": round(rd, 3), "GBps": round(fp.active_bytes / (rd * 1e-6) / 1e9, 1),
            "frac_of_it": round(rd / f_mean, 4),
            "what": "bsg_read_calibrate streaming the same bytes per launch (weight-load pattern, no compute), "
                    "same rotation and timing"}
        log(f"practical read of {fp.active_bytes / 1e6:.2f} MB: {rd:.2f} us ({roofline['practical_read']['GBps']} GB/s)")
    dense_pt = next((p for p in points if p.dense and p.name.startswith("down_b16")), None)
    if dense_pt is not None and not args.only:
        mm = torch_mm_us(dense_pt)
        for row in out_points:
            if row["name"] == dense_pt.name:
                row["torch_mm_us"] = round(mm, 3)
        log(f"torch.mm (hipBLASLt) on {dense_pt.name}: {mm:.2f} us")
    cpu = None
    if not args.no_cpu and not args.only:
        log("cpu baseline ...")
        cpu = cpu_baseline(fp, args.cpu_seconds)
        for p, row in zip(points, out_points):
            row["cpu_us_per_gemm"] = round(cpu_point_us(p), 1)
            row["gpu_speedup_over_cpu"] = round(row["cpu_us_per_gemm"] / row["us_per_gemm"], 1)
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
        "data": "synthetic: numpy PCG64 seed 1234, W~N(0,0.02) stored [K,N], X~Laplace(0,0.05)/N(0,1), "
                "masks rng.choice sorted; weights rotated over >=1 GiB of copies",
        "config": {"workload": workload, "gemms_per_step": sum(p.copies for p in points),
                   "value_is": "active-weight bytes / timed seconds over all sweep points"},
        "points": out_points,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
