"""GPU parity of the per-step oracle-map replay (bench.py --workload perstep, the reference's
headline benchmark scripts/bench_perstep_actual_kernel_speedup.py): for every batch size of the
fixture, the first group-steps' maps give the distinct (shape, density) cases that bench.py times;
each case runs through the same calls (tuned plan for (B, N, nblk, na), bsa.gemm_packed) and is
checked against the oracle, as are the dense variants the speedups divide by."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from bsa_mi355x import replay
from helpers import assert_close
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "perstep_smaps.npz")
STEPS_PER_BATCH = 2


@pytest.fixture(scope="module")
def weights(dev):
    out = {}
    for i, (name, (k, n)) in enumerate(replay.SHAPES.items()):
        rng = np.random.default_rng(1234 + i)
        w_kn = rng.normal(0.0, 0.02, size=(k, n)).astype(np.float16)
        out[name] = (np.ascontiguousarray(w_kn.T), bsa.pack_weight(torch.from_numpy(w_kn).to(dev), layout="kn"))
    yield out
    out.clear()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("bt", [2, 4, 8, 16, 32, 64])
def test_perstep_cases_match_oracle(dev, weights, bt):
    fx = replay.load_maps(FIXTURE)
    cases = replay.cases_for_batches(fx, [bt], steps_per_batch=STEPS_PER_BATCH)[bt]
    assert cases, f"no group-step for B={bt}"
    densities = {t for _, t in cases}
    assert len(densities) >= 3, densities  # the maps span several densities
    rng = np.random.default_rng(bt)
    xs = {name: rng.normal(0, 1, size=(bt, k)).astype(np.float16) for name, (k, _) in replay.SHAPES.items()}
    for name, (k, n) in replay.SHAPES.items():
        w_nk, packed = weights[name]
        nblk = replay.nblk_of(name)
        xt = torch.from_numpy(xs[name]).to(dev)
        y = torch.empty(bt, n, dtype=torch.float16, device=dev)
        pl = bsa.resolve_plan(bt, n, nblk, nblk, dev, None, dense=True)
        bsa.gemm_packed(xt, packed, n, None, y, plan=pl, workspace_prefix=f"rp_dense_{name}")
        torch.cuda.synchronize()
        assert_close(y.float().cpu().numpy(), orc.gemm_ref(xs[name], w_nk, np.arange(nblk)), f"B={bt} {name} dense")
        for cname, tenths in cases:
            if cname != name:
                continue
            na = replay.active_count(tenths, nblk)
            idx = replay.random_blocks(rng, nblk, na)
            pl = bsa.resolve_plan(bt, n, nblk, na, dev, None)
            y.fill_(float("nan"))
            bsa.gemm_packed(xt, packed, n, torch.from_numpy(idx).to(dev), y, plan=pl, workspace_prefix=f"rp_{name}")
            torch.cuda.synchronize()
            assert_close(y.float().cpu().numpy(), orc.gemm_ref(xs[name], w_nk, idx),
                         f"B={bt} {name} density {tenths / 10} na={na} plan={pl.as_tuple()}")


@pytest.fixture(scope="module")
def step_graphs(dev):
    sg = replay.StepGraphs(dev)
    yield sg
    del sg
    torch.cuda.empty_cache()


@pytest.mark.parametrize("bt", [2, 16, 64])
def test_step_graph_matches_eager_and_oracle(dev, step_graphs, bt):
    """One group-step of the reference's maps as a single 224-GEMM graph (32 layers x q, k, v,
    o, gate, up, down, per-layer weights): every output of three replays equals the eager step
    bit for bit, and layers 0, 15 and 31 are within the BASELINE tolerance of the oracle; the
    dense step graph likewise on layer 0."""
    sg = step_graphs
    fx = replay.load_maps(FIXTURE)
    row = replay.batch_rows(fx, bt)[0]
    sg.set_batch(bt)
    lists = sg.step_lists(fx["smap_tenths"][row], np.random.default_rng(bt))
    assert sg.active_bytes(lists) < sg.active_bytes(None)
    sg.run(lists)
    torch.cuda.synchronize()
    eager = [[y.clone() for y in layer] for layer in sg.y]
    for li in (0, 15, 31):
        for pi, shape in enumerate(replay.PROJ_SHAPE):
            k, n = replay.SHAPES[shape]
            w_nk = np.ascontiguousarray(orc.tile_unpermute(sg.packed[li][pi].cpu().numpy(), n).reshape(-1, n)[:k].T)
            x = sg.x[shape].cpu().numpy()
            print(f"step graph B={bt} layer {li} proj {pi} na={lists[li][pi].numel()}", flush=True)
            assert_close(sg.y[li][pi].float().cpu().numpy(), orc.gemm_ref(x, w_nk, lists[li][pi].cpu().numpy()),
                         f"B={bt} layer {li} proj {pi}")
    g = sg.capture(lists)
    for r in range(3):
        for layer in sg.y:
            for y in layer:
                y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for li in range(sg.n_layers):
            for pi in range(len(replay.PROJ_SHAPE)):
                assert torch.equal(sg.y[li][pi].view(torch.int16), eager[li][pi].view(torch.int16)), (r, li, pi)
    del g
    gd = sg.capture(None)
    gd.replay()
    torch.cuda.synchronize()
    for pi, shape in enumerate(replay.PROJ_SHAPE):
        k, n = replay.SHAPES[shape]
        nb = replay.nblk_of(shape)
        w_nk = np.ascontiguousarray(orc.tile_unpermute(sg.packed[0][pi].cpu().numpy(), n).reshape(-1, n)[:k].T)
        assert_close(sg.y[0][pi].float().cpu().numpy(), orc.gemm_ref(sg.x[shape].cpu().numpy(), w_nk, np.arange(nb)),
                     f"dense B={bt} layer 0 proj {pi}")
    del gd
