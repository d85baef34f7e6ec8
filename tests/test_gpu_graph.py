"""Graph capture: GEMM, split-K GEMM and fused select+GEMM recorded into a hipGraph (via
torch.cuda.CUDAGraph) and replayed several times, with eager work and synchronisations in
between; every replay must equal the eager result bit for bit (the kernels are deterministic
and leave their arrival counters at zero, so no memset node is needed)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from helpers import case, to_dev

pytestmark = pytest.mark.gpu


def _replays_match(fn, out, n_replays=4):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up: packs the weight, allocates the workspace
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    for r in range(n_replays):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {r} differs from eager"
        fn()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"eager after replay {r} differs"


@pytest.mark.parametrize("split_k", [1, 6])
def test_graph_gemm(dev, split_k):
    bt, k, n, na = 16, 11008, 4096, 62
    x, w_nk, idx = case(21, bt, k, n, na)
    xt = to_dev(x, dev).view(bt, 1, k)
    wt = to_dev(w_nk, dev)
    it = to_dev(idx, dev)
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    _replays_match(lambda: bsa._prepacked_block_sparse_gemm_from_active_blocks_splitk(
        xt, wt, it, out, cache_prefix=f"graph{split_k}", num_split_k=split_k), out)


def test_graph_bitmap_gemm(dev):
    bt, k, n, na = 64, 4096, 11008, 31
    x, w_nk, idx = case(22, bt, k, n, na, "normal")
    xt = to_dev(x, dev).view(bt, 1, k)
    wt = to_dev(w_nk, dev)
    it = to_dev(idx, dev)
    bm = bsa._build_active_k_bitmap(it, 64, dev)
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    _replays_match(lambda: bsa._prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk(
        xt, wt, it, out, cache_prefix="graph_bm", total_k_blocks=64, prebuilt_bitmap=bm, num_split_k=4), out)


def test_graph_select_gemm(dev):
    bt, k, n = 64, 4096, 11008
    x, w_nk, _ = case(23, bt, k, n, 1, "normal")
    xt = to_dev(x, dev).view(bt, 1, k)
    wt = to_dev(w_nk, dev)
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    idx_buf = torch.empty(31, dtype=torch.int32, device=dev)
    cnt_buf = torch.empty(1, dtype=torch.int32, device=dev)
    _replays_match(lambda: bsa.select_sparse_gemm(xt, wt, out, 31, cache_prefix="graph_sel", idx_out=idx_buf,
                                                  count_out=cnt_buf), out)
    assert int(cnt_buf.item()) == 31
    assert np.all(np.diff(idx_buf.cpu().numpy()) > 0)


def test_graph_dropin_with_in_kernel_sort(dev):
    """The reference's runtime entry with an unsorted list (sorted inside the GEMM's staging)
    captured and replayed: every replay and every eager call in between equal the first eager
    result bit for bit."""
    bt, k, n, na = 16, 11008, 4096, 86
    x, w_nk, idx = case(24, bt, k, n, na)
    xt = to_dev(x, dev).view(bt, 1, k)
    wt = to_dev(w_nk, dev)
    it = to_dev(np.random.default_rng(3).permutation(idx).astype(np.int32), dev)
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    _replays_match(lambda: bsa._prepacked_block_sparse_gemm_from_active_blocks(
        xt, wt, it, out, cache_prefix="graph_sort"), out)


def test_graph_one_launch_select_gemm(dev):
    """Selection + GEMM at B=2 (the GEMM scores the blocks itself: one launch) in a graph."""
    bt, k, n = 2, 4096, 4096
    x, w_nk, _ = case(25, bt, k, n, 1, "normal")
    xt = to_dev(x, dev).view(bt, 1, k)
    wt = to_dev(w_nk, dev)
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    idx_buf = torch.empty(13, dtype=torch.int32, device=dev)
    cnt_buf = torch.empty(1, dtype=torch.int32, device=dev)
    _replays_match(lambda: bsa.select_sparse_gemm(xt, wt, out, 13, cache_prefix="graph_sel1", idx_out=idx_buf,
                                                  count_out=cnt_buf), out)
    assert int(cnt_buf.item()) == 13
    from oracle import bsg_oracle as orc
    assert np.array_equal(idx_buf.cpu().numpy(), orc.select_topk_l1(x, 13))
