"""First-call tuning on the GPU (the reference's Triton autotune on (N_OUT, M, BATCHSIZE,
NUM_ACTIVE_BLOCKS), KRN:684-687): an untabled problem is tuned once on its own call's buffers,
later calls reuse the winner and `best_config` reports it; a tabulated problem never tunes; a
stream capture never tunes (heuristic plan, replay checked against the oracle)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from bsa_mi355x import autotune
from helpers import assert_close, case, to_dev
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture
def tuner():
    saved = dict(autotune._STATE)
    autotune.clear()
    autotune.set_autotune(True)
    yield autotune
    autotune.clear()
    autotune._STATE.clear()
    autotune._STATE.update(saved)


def _call(dev, x, w_nk, idx, prefix):
    bt, k = x.shape
    n = w_nk.shape[0]
    out = torch.full((bt, 1, n), float("nan"), dtype=torch.float16, device=dev)
    bsa._prepacked_block_sparse_gemm_from_active_blocks(to_dev(x, dev).view(bt, 1, k), to_dev(w_nk, dev),
                                                        to_dev(idx, dev), out, cache_prefix=prefix)
    torch.cuda.synchronize()
    return out.view(bt, n).float().cpu().numpy()


@pytest.mark.parametrize("bt,k,n,na", [(5, 2048, 1000, 7), (24, 3072, 640, 19), (48, 1024, 2000, 9)])
def test_untabled_problem_is_tuned_once(dev, tuner, bt, k, n, na):
    x, w_nk, idx = case(500 + bt, bt, k, n, na, "normal")
    ref = orc.gemm_ref64(x, w_nk, idx)
    assert_close(_call(dev, x, w_nk, idx, f"at{bt}"), ref, "first call (tuned)")
    st = tuner.stats()
    assert st["tunes"] == 1 and st["keys"] == 1 and st["timed_launches"] > 0
    key = autotune.key(n, orc.nblk_of(k), bt, na, "list", 0)
    plan = tuner.cached(key)
    cfg = bsa.prepacked_block_sparse_gemm_batched_kernel.best_config
    assert cfg.kwargs["BLOCK_B"] == plan.rows_per_group and cfg.num_warps == plan.waves_per_group
    assert cfg.num_stages == plan.depth and cfg.split_k == plan.split_k and cfg.kind == plan.kind
    assert_close(_call(dev, x, w_nk, idx, f"at{bt}"), ref, "second call (cached plan)")
    assert tuner.stats()["tunes"] == 1
    # another active-block count is another key
    idx2 = idx[: max(1, na - 2)]
    assert_close(_call(dev, x, w_nk, idx2, f"at{bt}"), orc.gemm_ref64(x, w_nk, idx2), "new key")
    assert tuner.stats()["tunes"] == 2


def test_tabulated_problem_is_not_tuned(dev, tuner):
    bt, k, n, na = 16, 11008, 4096, 86
    x, w_nk, idx = case(600, bt, k, n, na)
    assert_close(_call(dev, x, w_nk, idx, "at_tab"), orc.gemm_ref64(x, w_nk, idx), "tabulated")
    assert tuner.stats()["tunes"] == 0


def test_capture_never_tunes(dev, tuner):
    bt, k, n, na = 6, 2048, 700, 11
    x, w_nk, idx = case(700, bt, k, n, na, "normal")
    xt, it = to_dev(x, dev), to_dev(idx, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    y = torch.full((bt, n), float("nan"), dtype=torch.float16, device=dev)
    # warm the heuristic plan's workspace outside the capture, with tuning off
    autotune.set_autotune(False)
    bsa.gemm_packed(xt, packed, n, it, y, workspace_prefix="at_cap")
    torch.cuda.synchronize()
    autotune.set_autotune(True)
    y.fill_(float("nan"))
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            bsa.gemm_packed(xt, packed, n, it, y, workspace_prefix="at_cap")
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    assert tuner.stats()["tunes"] == 0
    ref = orc.gemm_ref64(x, w_nk, idx)
    for _ in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert_close(y.float().cpu().numpy(), ref, "captured heuristic plan")
    # an eager call afterwards tunes the key
    bsa.gemm_packed(xt, packed, n, it, y, workspace_prefix="at_cap")
    torch.cuda.synchronize()
    assert tuner.stats()["tunes"] == 1
    assert_close(y.float().cpu().numpy(), ref, "eager after capture (tuned)")
