"""Host-side logic without a GPU: tuned-plan lookup, the reference's lookup-table schemas,
reference tile -> plan mapping, and the drop-in module path."""
from __future__ import annotations

import ctypes
import json
import os

import pytest

import bsa_mi355x as bsa
from bsa_mi355x import tuning


def test_shipped_table_covers_baseline_shapes():
    entries = tuning.load_table()
    assert entries, "tuned_plans.json missing or empty"
    shapes = {(e["N"], e["K"]) for e in entries}
    assert {(4096, 4096), (11008, 4096), (4096, 11008)} <= shapes
    assert {e["bt"] for e in entries} >= {2, 16, 64}
    assert any(e["dense"] for e in entries)
    lib = bsa.load()
    for e in entries:
        assert len(e["plan"]) == 6 and e["plan"][0] >= 1 and e["plan"][5] in (1, 2, 3, 4, 5, 6, 7)
        # every shipped plan names an instantiated kernel the library accepts as is
        p = bsa.Plan(*e["plan"])
        want = p.as_tuple()
        assert lib.bsg_plan_resolve(e["bt"], e["N"], -(-e["K"] // 64), e["na"], 256, ctypes.byref(p)) == 0, e
        assert p.as_tuple() == want, (e, p.as_tuple())


def test_lookup_nearest_batch_and_density():
    tuning.load_table()
    p = tuning.lookup(16, 4096, 172, 86)
    assert p is not None and p.rows_per_group == 16
    assert tuning.lookup(64, 11008, 64, 31).rows_per_group == 64
    assert tuning.lookup(8, 4096, 172, 80) is not None        # nearest batch in the 16-row bucket
    assert tuning.lookup(16, 1234, 172, 86) is None           # shape not tabulated
    d = tuning.lookup(16, 4096, 172, 172, dense=True)
    assert d is not None


def test_lookup_from_custom_table(tmp_path):
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"entries": [
        {"bt": 16, "N": 100, "K": 640, "na": 3, "dense": False, "plan": [2, 16, 4, 4, 16, 1], "us": 1.0},
        {"bt": 16, "N": 100, "K": 640, "na": 8, "dense": False, "plan": [1, 32, 2, 4, 16, 1], "us": 1.0},
    ]}))
    tuning.load_table(str(path))
    try:
        assert tuning.lookup(16, 100, 10, 4).as_tuple() == (2, 16, 4, 4, 16, 1)
        assert tuning.lookup(16, 100, 10, 7).as_tuple() == (1, 32, 2, 4, 16, 1)
        assert tuning.lookup(64, 100, 10, 7) is None          # no 64-row entry
    finally:
        tuning.load_table()


class _ScriptedCase:
    """Stands in for tuning._Case: each plan returns its scripted timings in turn."""

    def __init__(self, times):
        self.times = {k: list(v) for k, v in times.items()}
        self.calls = []
        self.selects = []

    def time(self, plan, dense=False, select=False):
        key = plan.as_tuple()
        self.calls.append(key)
        self.selects.append(select)
        v = self.times[key].pop(0)
        if v is None:
            raise bsa.BsgUnsupported(-5, "not instantiated")
        return v


def test_tuner_retimes_close_candidates():
    a, b, c, d = (bsa.Plan(1, 16, 2, 4, 16, 1), bsa.Plan(1, 16, 4, 4, 16, 1), bsa.Plan(2, 32, 2, 4, 16, 1),
                  bsa.Plan(1, 64, 2, 4, 16, 1))
    # b's single first timing is lucky; a is faster on the median of four; c is out of the 5%
    # margin and never re-timed; d is rejected by the library
    case = _ScriptedCase({a.as_tuple(): [5.0, 4.8, 4.9, 4.85], b.as_tuple(): [4.9, 5.6, 5.5, 5.7],
                          c.as_tuple(): [6.0], d.as_tuple(): [None]})
    us, plan = tuning._pick(case, [a, b, c, d])
    assert plan.as_tuple() == a.as_tuple() and us == pytest.approx(4.875)
    assert case.calls.count(c.as_tuple()) == 1 and case.calls.count(b.as_tuple()) == 4
    # a lone finalist is taken on its first timing; nothing runnable gives (inf, None)
    case = _ScriptedCase({a.as_tuple(): [5.0], c.as_tuple(): [6.0]})
    assert tuning._pick(case, [a, c]) == (5.0, a)
    assert tuning._pick(_ScriptedCase({d.as_tuple(): [None]}), [d]) == (float("inf"), None)
    # the selection + GEMM tuning times every candidate through the select path
    case = _ScriptedCase({a.as_tuple(): [5.0, 4.8, 4.9, 4.85], b.as_tuple(): [4.9, 5.6, 5.5, 5.7]})
    tuning._pick(case, [a, b], select=True)
    assert case.selects and all(case.selects)


def test_lookup_prefers_select_entries_for_select_gemm(tmp_path):
    """Entries timed as selection + GEMM ("select": true) answer select lookups first and never
    plain-GEMM lookups; a select lookup with no select entry in its row bucket falls back to the
    plain GEMM's entries."""
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"entries": [
        {"bt": 64, "N": 4096, "K": 11008, "na": 86, "dense": False, "plan": [4, 16, 4, 4, 64, 2], "us": 1.0},
        {"bt": 64, "N": 4096, "K": 11008, "na": 86, "dense": False, "select": True, "plan": [4, 16, 8, 4, 64, 4],
         "us": 1.0},
        {"bt": 16, "N": 4096, "K": 11008, "na": 86, "dense": False, "plan": [2, 32, 2, 4, 16, 1], "us": 1.0},
        {"bt": 64, "N": 4096, "K": 11008, "na": 172, "dense": True, "plan": [8, 16, 8, 4, 64, 2], "us": 1.0},
    ]}))
    tuning.load_table(str(path))
    try:
        assert tuning.lookup(64, 4096, 172, 83).as_tuple() == (4, 16, 4, 4, 64, 2)
        assert tuning.lookup(64, 4096, 172, 83, select=True).as_tuple() == (4, 16, 8, 4, 64, 4)
        assert tuning.lookup(16, 4096, 172, 83, select=True).as_tuple() == (2, 32, 2, 4, 16, 1)
        assert tuning.lookup(64, 4096, 172, 172, dense=True, select=True).as_tuple() == (8, 16, 8, 4, 64, 2)
    finally:
        tuning.load_table()


def test_lookup_row_groups_only_as_tuned(tmp_path):
    """A 64-row-bucket batch may run two 32-row groups (tuned so); a 16-row tile never serves
    a larger batch."""
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"entries": [
        {"bt": 64, "N": 4096, "K": 4096, "na": 30, "dense": False, "plan": [1, 32, 2, 4, 32, 1], "us": 1.0},
        {"bt": 64, "N": 4096, "K": 4096, "na": 40, "dense": False, "plan": [1, 16, 2, 4, 16, 1], "us": 1.0},
    ]}))
    tuning.load_table(str(path))
    try:
        assert tuning.lookup(64, 4096, 64, 30).as_tuple() == (1, 32, 2, 4, 32, 1)
        assert tuning.lookup(48, 4096, 64, 30).as_tuple() == (1, 32, 2, 4, 32, 1)
        assert tuning.lookup(64, 4096, 64, 40) is None
        assert tuning.lookup(32, 4096, 64, 40) is None        # no 32-row-bucket entry
    finally:
        tuning.load_table()
    assert {p.rows_per_group for p in tuning.candidate_plans(64, 30, 64)} == {32, 64}
    assert {p.rows_per_group for p in tuning.candidate_plans(32, 30, 64)} == {16, 32, 64}
    assert {p.rows_per_group for p in tuning.candidate_plans(16, 30, 64)} == {16}


def test_reference_lookup_both_key_sets(tmp_path):
    pkc = {"down": {"0.5": {"mask": "bitmap", "block_k": 64, "K": 4, "tile": [16, 64, 2, 3],
                            "dense_ms": 0.05, "sparse_ms": 0.03, "speedup": 1.6},
                    "1.0": {"mask": "dense", "K": 1, "tile": None}}}
    rrd = {"down": {"0.5": {"best_kern": "naive", "best_K": 2, "best_tile": [32, 128, 4, 2]}}}
    p1 = tmp_path / "llama2_kernel_best_sweep_B16.json"
    p1.write_text(json.dumps(pkc))
    p2 = tmp_path / "rrd.json"
    p2.write_text(json.dumps(rrd))
    a = tuning.load_reference_lookup(str(p1))
    b = tuning.load_reference_lookup(str(p2))
    key, cfg = tuning.nearest_density_cfg(a["down"], 0.47)
    assert key == 0.5 and cfg["mask"] == "bitmap"
    assert tuning.plan_from_reference_cfg(cfg, bt=16).as_tuple() == (4, 64, 2, 4, 16, 0)
    assert tuning.plan_from_reference_cfg(a["down"][1.0], bt=16) is None
    cfg_b = b["down"][0.5]
    assert cfg_b["mask"] == "naive" and cfg_b["K"] == 2
    assert tuning.plan_from_reference_cfg(cfg_b, bt=16).as_tuple() == (2, 128, 4, 2, 32, 0)
    own = {"plan": [3, 16, 4, 4, 64, 2], "mask": "naive", "K": 3}
    assert tuning.plan_from_reference_cfg(own, bt=64).as_tuple() == (3, 16, 4, 4, 64, 2)


def test_dropin_module_path_exports_reference_names():
    from kernels.shared_mask_batched_triton_min_runtime import (  # noqa: F401
        INDEX_BLOCK_META_SIZE, _PREPACK_AUTOTUNE_CONFIGS, _build_active_k_bitmap, _get_prepacked_weight_block_major,
        _prepacked_block_sparse_gemm_from_active_blocks,
        _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload,
        _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk,
        _prepacked_block_sparse_gemm_from_active_blocks_splitk, prepacked_block_sparse_gemm_batched_kernel,
        prepacked_block_sparse_gemm_bitmap_preload_batched_kernel)
    assert INDEX_BLOCK_META_SIZE == 64
    assert prepacked_block_sparse_gemm_bitmap_preload_batched_kernel.best_config is None
    cfg = _PREPACK_AUTOTUNE_CONFIGS[0]
    assert cfg.kwargs["BLOCK_B"] in (16, 32, 64) and cfg.num_warps in (1, 2, 4, 8)


def test_cpu_tensors_are_rejected():
    import torch

    x = torch.zeros(2, 1, 64, dtype=torch.float16)
    w = torch.zeros(16, 64, dtype=torch.float16)
    out = torch.zeros(2, 1, 16, dtype=torch.float16)
    with pytest.raises(ValueError):
        bsa._prepacked_block_sparse_gemm_from_active_blocks(x, w, torch.tensor([0], dtype=torch.int32), out)


def test_bench_traffic_profile_per_roofline_point():
    """Each workload's roofline point reads the PMC summary of that same point, and the figure
    is at least the point's algorithmic bytes (active weight na*64*N*2)."""
    import importlib.util

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    algorithmic = {"down_b16_s500": 86 * 64 * 4096 * 2, "gate_up_b64_s520": 31 * 64 * 11008 * 2,
                   "gate_up_b16_s638": 23 * 64 * 11008 * 2}
    assert set(bench.TRAFFIC_PROFILES) == set(algorithmic)
    for point, path in bench.TRAFFIC_PROFILES.items():
        assert point.split("_s")[0].replace("_", "") in os.path.basename(path).replace("_", "")
        t = bench.load_traffic(point)
        assert isinstance(t, int) and algorithmic[point] <= t < 1.2 * algorithmic[point], (point, t)
    assert bench.load_traffic("qkvo_b2_s803") is None


def test_bench_roofline_profiles_match_the_tuned_kernel():
    """The committed traffic and counter summaries of the llama roofline points (the dominant
    kernel's largest sparse launch, gate/up B=16 s=0.638 with the shipped plans; the CPU-reference
    point, down B=16 s=0.5; configs[3]'s GEMM, gate/up B=64 s=0.52) were taken on
    the kernel their tuned plans launch now (a retune that changes the kernel makes them stale)."""
    bench = _bench_module()
    from bsa_mi355x import tuning

    for point, (bt, n, nblk, na) in (("gate_up_b64_s520", (64, 11008, 64, 31)),
                                     ("gate_up_b16_s638", (16, 11008, 64, 23)),
                                     ("down_b16_s500", (16, 4096, 172, 86))):
        plan = tuning.lookup(bt, n, nblk, na)
        assert plan is not None
        kern = bench.KERNEL_NAMES[plan.kind]
        for prof in (bench.TRAFFIC_PROFILES[point], bench.MFMA_PROFILES[point]):
            with open(prof) as f:
                text = f.read()
            assert kern in text, (prof, kern)
            assert ",".join(str(v) for v in plan.as_tuple()) in text.replace(" ", ""), (prof, plan)
        mf = bench.load_mfma_util(point)
        assert mf is not None and 0.0 < mf["value"] < 1.0
    assert bench.load_mfma_util("qkvo_b2_s803") is None


class _P:
    def __init__(self, name, kind, copies, active, dense=False):
        self.name, self.copies, self.active_bytes, self.dense = name, copies, active, dense
        self.plan = bsa.Plan(1, 16, 2, 4, 16, kind)


def test_bench_roofline_point_is_the_dominant_kernels_largest_sparse_launch():
    """The roofline goes on the kernel with the largest share of the step's GPU time, at its
    sparse point with the most active-weight bytes per launch."""
    bench = _bench_module()
    pts = [_P("down_b16_s500", 1, 10, 45), _P("down_b16_dense", 1, 5, 90, dense=True),
           _P("qkvo_b2_s803", 6, 100, 7), _P("gate_up_b64_s520", 6, 20, 44)]
    per = {"down_b16_s500": (11.0, 11.0), "down_b16_dense": (17.0, 17.0), "qkvo_b2_s803": (3.6, 3.6),
           "gate_up_b64_s520": (13.7, 13.7)}
    shares = bench.kernel_shares(pts, per)
    assert next(iter(shares)) == "bsg_gemm_vt_kernel" and shares["bsg_gemm_vt_kernel"]["top_point"] == "qkvo_b2_s803"
    assert bench.roofline_point(pts, shares) == "gate_up_b64_s520"
    per["down_b16_s500"] = (80.0, 80.0)  # kind 1 now dominates the step
    shares = bench.kernel_shares(pts, per)
    assert bench.roofline_point(pts, shares) == "down_b16_s500"  # its largest sparse launch, not the dense one


def _bench_module():
    import importlib.util

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    return bench


def test_bench_default_measures_configs2_with_active_byte_rotation():
    """The default workload is BASELINE configs[2] (three projection shapes x B=2@0.803,
    16@0.638, 64@0.520, each with a dense point) plus the configs[1] sweep, and every point's
    graph reads >= 1 GiB of distinct ACTIVE weight (copies sized on active, not packed, bytes)."""
    bench = _bench_module()
    rows = bench.matrix_points("llama", None)
    names = {r[0] for r in rows}
    for sh in ("qkvo", "gate_up", "down"):
        for b, s in ((2, "s803"), (16, "s638"), (64, "s520")):
            assert f"{sh}_b{b}_{s}" in names and f"{sh}_b{b}_dense" in names
    assert {"down_b16_s250", "down_b16_s500", "down_b16_s800"} <= names
    assert dict((r[0], r[3]) for r in rows)["gate_up_b64_s520"] == 31
    need = bench.pool_copies(rows)
    for name, sh, bt, na, dense in rows:
        k, n = bench.SHAPES[sh]
        active = na * 64 * n * 2
        copies = min(need[sh], bench.copies_for(active))
        assert copies * active >= 1 << 30, (name, copies, active)
    assert bench.KERNEL_NAMES[4] == "bsg_gemm_xl_kernel"
    assert set(bench.KERNEL_NAMES) == {1, 2, 3, 4, 5, 6, 7}


def test_bench_default_line_carries_configs3_configs4_and_the_perstep_table(monkeypatch):
    """With no flags, bench.py runs the llama matrix and, in the same run, the fused select +
    GEMM, the 32-layer decode step and the per-step replay at every batch
    size of the reference's fixture; --no-extras and --only skip them."""
    bench = _bench_module()
    monkeypatch.setattr("sys.argv", ["bench.py"])
    a = bench.parse_args()
    assert (a.workload, a.gpus, a.no_extras, a.only, a.layers) == ("llama", 1, False, None, 32)
    monkeypatch.setattr("sys.argv", ["bench.py", "--no-extras"])
    assert bench.parse_args().no_extras
    from bsa_mi355x import replay

    fx = replay.load_maps(bench.PERSTEP_FIXTURE)
    assert sorted(int(b) for b in fx["ref_batch"]) == [2, 4, 8, 16, 32, 64]


def test_reference_prior_length_rule_on_the_host():
    """The drop-in selectors pass a block prior on only when it holds floor(K/64) entries
    (RRD:110-112): shorter and longer priors are dropped before any device call."""
    import torch

    from bsa_mi355x.select import _prior_or_none

    x = torch.zeros(4, 1, 4096 + 32, dtype=torch.float16)  # floor(4128 / 64) = 64 scored blocks
    for n in (63, 65, 1, 128):
        assert _prior_or_none(torch.ones(n), x) is None
    p = torch.ones(64)
    assert _prior_or_none(p, x) is p
    assert _prior_or_none(None, x) is None


def test_tiled_packed_weight_block_major_matches_the_reference_packing():
    """TiledPackedWeight (what _get_prepacked_weight_block_major returns) undoes the tile order
    exactly: block_major(N) of tile_permute(pack_kmajor(W)) is pack_kmajor(W) (KRN:3152-3162),
    including a K tail and an N that is not a multiple of 16; reference-layout indexing raises."""
    import numpy as np
    import torch

    from oracle import bsg_oracle as orc
    from bsa_mi355x.runtime import TiledPackedWeight

    for n, k in ((100, 1000), (48, 64), (37, 200)):
        w = np.random.default_rng(n * k).normal(0, 0.02, size=(n, k)).astype(np.float16)
        ref = orc.pack_kmajor(w)
        tp = torch.from_numpy(orc.tile_permute(ref)).as_subclass(TiledPackedWeight)
        assert np.array_equal(tp.block_major(n).numpy().view(np.uint16), ref.view(np.uint16)), (n, k)
        with pytest.raises(TypeError):
            tp[0, :, :n]
        assert "TiledPackedWeight" in repr(tp)


def test_bench_kernel_shares_weight_points_by_launches_per_step():
    """roofline.by_kernel: each kernel's share of a step's time (a point's mean µs x its launches
    per step) and its active bytes over that time."""
    import types

    bench = _bench_module()
    P = types.SimpleNamespace
    pts = [P(name="a", plan=P(kind=1), copies=10, active_bytes=1_000_000),
           P(name="b", plan=P(kind=6), copies=5, active_bytes=4_000_000),
           P(name="c", plan=P(kind=1), copies=2, active_bytes=9_000_000)]
    per = {"a": (3.0, 3.0), "b": (10.0, 10.0), "c": (15.0, 15.0)}
    out = bench.kernel_shares(pts, per)
    assert list(out) == ["bsg_gemm_kernel", "bsg_gemm_vt_kernel"]  # 60 µs vs 50 µs per step
    k1 = out["bsg_gemm_kernel"]
    assert k1["points"] == ["a", "c"] and abs(k1["time_share"] - 60 / 110) < 1e-4
    assert abs(k1["GBps"] - 28_000_000 / 60e-6 / 1e9) < 0.1
    assert abs(out["bsg_gemm_vt_kernel"]["frac"] - (20_000_000 / 50e-6 / 1e9) / bench.HBM_PEAK_GBS) < 1e-4
