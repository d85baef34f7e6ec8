"""GPU parity of the fused L1 block selector: indices must be bit-exact vs the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from helpers import assert_close, case, to_dev
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu


def _select(dev, x, k):
    idx, cnt = bsa.select_topk_l1(to_dev(x, dev), k)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), int(cnt.item())


@pytest.mark.parametrize("bt,kdim,k", [(1, 64, 1), (2, 4096, 13), (16, 4096, 23), (64, 4096, 31), (16, 11008, 62),
                                       (64, 11008, 83), (5, 1000, 7), (3, 128000, 900), (64, 4096, 64),
                                       (64, 4096, 100)])
def test_select_matches_oracle(dev, bt, kdim, k):
    rng = np.random.default_rng(bt * 7 + k)
    x = rng.laplace(0, 0.05, size=(bt, kdim)).astype(np.float16)
    got, cnt = _select(dev, x, k)
    want = orc.select_topk_l1(x, k)
    assert cnt == len(want)
    assert np.array_equal(got, want)


def test_select_ties_go_to_lower_index(dev):
    bt, kdim = 8, 4096
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, size=(bt, kdim)).astype(np.float16)
    # blocks 10, 20, 30 identical (equal scores), and the strongest
    for j in (10, 20, 30):
        x[:, 64 * j:64 * j + 64] = 50.0
    got, _ = _select(dev, x, 2)
    assert np.array_equal(got, [10, 20])
    assert np.array_equal(got, orc.select_topk_l1(x, 2))
    # all-zero input: every score ties at 0 -> the k lowest ids
    z = np.zeros((bt, kdim), dtype=np.float16)
    got, _ = _select(dev, z, 5)
    assert np.array_equal(got, np.arange(5))


def test_select_extreme_values(dev):
    """Largest finite fp16, subnormals and negative zeros are scored exactly."""
    bt, kdim = 64, 4096
    x = np.zeros((bt, kdim), dtype=np.float16)
    x[:, 64 * 3:64 * 4] = np.float16(65504.0)
    x[:, 64 * 7:64 * 8] = -np.float16(65504.0)
    x[0, 64 * 9] = np.float16(2.0 ** -24)
    x[1, 64 * 11] = -np.float16(0.0)
    x[2, 64 * 12:64 * 13] = np.float16(2.0 ** -20)
    got, _ = _select(dev, x, 4)
    assert np.array_equal(got, orc.select_topk_l1(x, 4))
    assert np.array_equal(got, [3, 7, 9, 12])


@pytest.mark.parametrize("shape,bt,k", [((4096, 11008), 64, 31), ((11008, 4096), 16, 62), ((4096, 4096), 2, 13)])
def test_fused_select_gemm(dev, shape, bt, k):
    """fused selection at k then the sparse GEMM on the device list."""
    kdim, n = shape
    x, w_nk, _ = case(1234, bt, kdim, n, 1, "normal")
    xt = to_dev(x, dev).view(bt, 1, kdim)
    out = torch.empty(bt, 1, n, dtype=torch.float16, device=dev)
    idx, cnt = bsa.select_sparse_gemm(xt, to_dev(w_nk, dev), out, k)
    torch.cuda.synchronize()
    want = orc.select_topk_l1(x, k)
    assert np.array_equal(idx.cpu().numpy(), want)
    assert int(cnt.item()) == k
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), "fused select+gemm")


def test_select_density_wrapper(dev):
    x = np.random.default_rng(9).normal(0, 1, size=(64, 4096)).astype(np.float16)
    got = bsa._select_active_blocks_l1(to_dev(x, dev).view(64, 1, 4096), 0.48)
    torch.cuda.synchronize()
    assert got.dtype == torch.int32 and got.numel() == orc.n_keep(0.48, 64) == 31
    assert np.array_equal(got.cpu().numpy(), orc.select_topk_l1(x, 31))
