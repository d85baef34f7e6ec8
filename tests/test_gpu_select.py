"""GPU parity of the fused L1 block selector: indices must be bit-exact vs the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from bsa_mi355x.select import select_gemm_packed
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


def _fused(dev, x, w_nk, k, plan=None):
    bt, kdim = x.shape
    n = w_nk.shape[0]
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    y = torch.empty(bt, n, dtype=torch.float16, device=dev)
    idx, cnt = select_gemm_packed(to_dev(x, dev), packed, n, k, y,
                                  plan=None if plan is None else bsa.Plan(*plan), workspace_prefix="t_fused")
    torch.cuda.synchronize()
    c = int(cnt.item())
    return idx.cpu().numpy()[:c], c, y.float().cpu().numpy()


@pytest.mark.parametrize("bt,kdim,n,k,plan", [
    (64, 4096, 11008, 31, (1, 16, 8, 4, 64, 4)),  # channel-half waves; ranked in the GEMM
    (64, 4096, 4096, 31, (2, 16, 4, 4, 64, 2)),   # X tile in LDS, split-K 2; in the GEMM
    (64, 11008, 4096, 83, (4, 16, 8, 4, 64, 4)),  # 172 blocks over 8 waves; in the GEMM
    (64, 11008, 4096, 83, (4, 16, 4, 4, 64, 2)),  # 172 blocks over 4 waves (9 rank items each); in the GEMM
    (16, 4096, 4096, 23, (1, 16, 1, 4, 16, 1)),   # one wave ranks 64 blocks; in the GEMM
    (16, 11008, 4096, 86, (1, 16, 2, 4, 16, 1)),  # 172 blocks, 2 waves: rank launch, then the list
    (2, 4096, 4096, 13, (1, 16, 4, 4, 2, 3)),     # dot-product kernel: rank launch, then the list
    (80, 4096, 1024, 20, None),                   # > 64 rows: pair compares, two grid rows
    (8, 32768, 256, 100, (1, 16, 1, 4, 16, 1)),   # 512 blocks: rank launch
    (4, 38400, 256, 77, None),                    # 600 blocks: rank launch
    (16, 4096, 512, 0, None), (16, 4096, 512, 64, None), (16, 4096, 512, 200, None),
    (64, 4096, 11008, 31, (1, 48, 2, 4, 64, 6)),  # variable-width groups, waves split blocks
    (16, 4096, 12288, 23, (1, 48, 4, 4, 16, 5)),  # variable-width groups, channel-half waves
    (64, 4096, 22016, 31, (1, 96, 2, 4, 64, 5)),  # 5-6 subtiles per group
    (64, 4096, 11008, 31, (1, 48, 4, 2, 64, 7)),  # activations through LDS
    (64, 4096, 12288, 31, (1, 48, 8, 2, 64, 7)),  # eight block-slice waves
    (64, 11008, 4096, 83, (1, 32, 4, 2, 32, 7)),  # 172 blocks, two 32-row groups
    (16, 4096, 4096, 23, (1, 32, 4, 4, 16, 7)),
    (2, 4096, 4096, 13, (1, 32, 4, 4, 16, 7)),    # the work-groups score the blocks themselves
])
def test_fused_select_gemm_every_kind(dev, bt, kdim, n, k, plan):
    """Selection + GEMM for every kernel kind and edge k, with the top-k either ranked inside
    the GEMM's work-groups or by a separate rank launch (the library picks by plan); the kept
    list and count are published either way."""
    x, w_nk, _ = case(4321 + bt + k, bt, kdim, n, 1, "normal")
    got, c, y = _fused(dev, x, w_nk, k, plan)
    want = orc.select_topk_l1(x, k)
    assert c == len(want) == min(k, -(-kdim // 64))
    assert np.array_equal(got, want)
    assert_close(y, orc.gemm_ref(x, w_nk, want), f"fused bt={bt} K={kdim} k={k} plan={plan}")


def test_fused_select_gemm_ties_and_repeats(dev):
    """Equal scores go to the lower index inside the GEMM's own ranking, and a second call on
    new activations (same workspace) selects afresh."""
    bt, kdim, n = 8, 4096, 256
    x, w_nk, _ = case(77, bt, kdim, n, 1, "normal")
    for j in (10, 20, 30):
        x[:, 64 * j:64 * j + 64] = 50.0
    got, c, y = _fused(dev, x, w_nk, 2)
    assert c == 2 and np.array_equal(got, [10, 20])
    assert_close(y, orc.gemm_ref(x, w_nk, [10, 20]), "fused ties")
    x2, _, _ = case(78, bt, kdim, n, 1, "normal")
    got2, c2, y2 = _fused(dev, x2, w_nk, 9)
    want2 = orc.select_topk_l1(x2, 9)
    assert c2 == 9 and np.array_equal(got2, want2)
    assert_close(y2, orc.gemm_ref(x2, w_nk, want2), "fused repeat")


SELF_CASES = [  # (bt, K, N, k, plan): bt x K x 2 <= 24 KiB, so the GEMM scores the blocks itself
    (1, 4096, 4096, 13, None), (2, 4096, 4096, 13, (1, 16, 4, 4, 16, 6)), (3, 4096, 11008, 31, (1, 16, 1, 4, 16, 1)),
    (5, 1000, 300, 7, None), (8, 1024, 1000, 5, (1, 48, 4, 4, 16, 5)), (8, 1536, 4096, 11, (2, 16, 8, 4, 16, 4)),
    (4, 3072, 4096, 20, (1, 16, 4, 4, 16, 6)), (1, 11008, 4096, 86, (2, 32, 4, 4, 16, 1)),
    (7, 1536, 512, 0, None), (6, 2048, 512, 64, None),
]


@pytest.mark.parametrize("bt,kdim,n,k,plan", SELF_CASES)
def test_self_scored_selection_in_one_launch(dev, bt, kdim, n, k, plan):
    """At bt <= 8 and bt x K x 2 <= 24 KiB the selection + GEMM is one launch: every GEMM
    work-group scores the blocks from x itself.  No score is written (the selector's part of the
    workspace keeps a planted pattern); indices and count are bit-exact against the oracle; Y is
    bit for bit the GEMM on the same list through bsg_gemm, and within tolerance of the oracle.
    x holds ties (three equal blocks), a block far above the rest, a subnormal and -0."""
    import ctypes

    from bsa_mi355x import _lib
    from bsa_mi355x.runtime import _stream_handle

    x, w_nk, _ = case(900 + bt + k, bt, kdim, n, 1, "normal")
    nb = -(-kdim // 64)
    for j in (1, 4, nb - 1):
        x[:, 64 * j:min(64 * j + 64, kdim)] = 7.0
    x[0, 64 * 2:64 * 3] = np.float16(2048.0)
    x[bt - 1, 64 * 3] = np.float16(2.0 ** -24)
    x[bt // 2, 64 * 5] = -np.float16(0.0)
    lib = bsa.load()
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    pl = bsa.resolve_plan(bt, n, nb, min(k, nb), dev, None if plan is None else bsa.Plan(*plan), select=True)
    sel = int(lib.bsg_select_workspace_bytes(kdim))
    gws = int(lib.bsg_gemm_workspace_bytes(bt, n, ctypes.byref(pl)))
    ws = torch.zeros(sel + gws, dtype=torch.uint8, device=dev)
    ws[256:sel] = 0xAB
    y = torch.full((bt, n), float("nan"), dtype=torch.float16, device=dev)
    idx = torch.full((max(k, 1),), -1, dtype=torch.int32, device=dev)
    cnt = torch.full((1,), -1, dtype=torch.int32, device=dev)
    print(f"self-scored select+gemm bt={bt} K={kdim} N={n} k={k} plan={pl.as_tuple()}", flush=True)
    rc = lib.bsg_select_gemm(xt.data_ptr(), kdim, bt, kdim, k, packed.data_ptr(), n, idx.data_ptr(), cnt.data_ptr(),
                             y.data_ptr(), n, 0, ws.data_ptr(), sel + gws, ctypes.byref(pl), _stream_handle(dev))
    assert rc == _lib.BSG_OK, _lib.last_error()
    torch.cuda.synchronize()
    assert bool((ws[256:sel] == 0xAB).all()), "a score launch ran"
    want = orc.select_topk_l1(x, k)
    c = int(cnt.item())
    assert c == len(want) == min(k, nb)
    assert np.array_equal(idx.cpu().numpy()[:c], want)
    y_list = torch.full((bt, n), float("nan"), dtype=torch.float16, device=dev)
    bsa.gemm_packed(xt, packed, n, to_dev(want.astype(np.int32), dev) if c else None, y_list,
                    num_active=c if c else None, plan=pl if c else None, workspace_prefix="t_self_ref")
    torch.cuda.synchronize()
    if c:
        assert torch.equal(y, y_list), "one-launch selection + GEMM differs from the GEMM on its list"
        assert_close(y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), f"self-scored bt={bt} K={kdim}")
    else:
        assert torch.count_nonzero(y).item() == 0


@pytest.mark.parametrize("bt,kdim,n,k,plan", [(3, 4096, 1024, 13, (1, 16, 4, 4, 16, 6)),
                                              (8, 1536, 4096, 11, (1, 48, 4, 4, 16, 5)),
                                              (2, 4096, 512, 5, (1, 16, 2, 4, 16, 1))])
def test_self_scored_selection_with_inf_and_nan(dev, bt, kdim, n, k, plan):
    """Non-finite activations on the one-launch path: the self-scored sums take the integer units
    for a group holding Inf or NaN (both above every finite value, NaN above Inf), which must
    rank exactly as the score launch's integer sums and the oracle do.  One +Inf and one NaN sit
    in different blocks and rows; the count and ids must equal the oracle's and the two-launch
    selector's (bsg_select_topk_l1) on the same x.  Y agrees with the GEMM on the same list: the
    same non-finite positions, and bit for bit (and within tolerance of the oracle) on the rows
    that hold neither value."""
    import ctypes

    from bsa_mi355x import _lib
    from bsa_mi355x.runtime import _stream_handle

    x, w_nk, _ = case(1700 + bt + k, bt, kdim, n, 1, "normal")
    nb = -(-kdim // 64)
    inf_row, inf_blk, nan_row, nan_blk = 0, 5, bt - 1, 9
    x[inf_row, 64 * inf_blk + 3] = np.float16(np.inf)
    x[nan_row, 64 * nan_blk + 7] = np.float16(np.nan)
    want = orc.select_topk_l1(x, k)
    assert inf_blk in want and nan_blk in want
    lib = bsa.load()
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    pl = bsa.Plan(*plan)
    sel = int(lib.bsg_select_workspace_bytes(kdim))
    gws = int(lib.bsg_gemm_workspace_bytes(bt, n, ctypes.byref(pl)))
    ws = torch.zeros(sel + gws, dtype=torch.uint8, device=dev)
    ws[256:sel] = 0xAB
    y = torch.full((bt, n), 1.0, dtype=torch.float16, device=dev)
    idx = torch.full((k,), -1, dtype=torch.int32, device=dev)
    cnt = torch.full((1,), -1, dtype=torch.int32, device=dev)
    print(f"self-scored select+gemm with Inf/NaN bt={bt} K={kdim} N={n} k={k} plan={plan}", flush=True)
    rc = lib.bsg_select_gemm(xt.data_ptr(), kdim, bt, kdim, k, packed.data_ptr(), n, idx.data_ptr(), cnt.data_ptr(),
                             y.data_ptr(), n, 0, ws.data_ptr(), sel + gws, ctypes.byref(pl), _stream_handle(dev))
    assert rc == _lib.BSG_OK, _lib.last_error()
    torch.cuda.synchronize()
    assert bool((ws[256:sel] == 0xAB).all()), "a score launch ran: the case is not the one-launch path"
    c = int(cnt.item())
    assert c == len(want) == min(k, nb)
    assert np.array_equal(idx.cpu().numpy()[:c], want)
    two_idx, two_cnt = _select(dev, x, k)
    assert two_cnt == c and np.array_equal(two_idx[:two_cnt], want)
    y_list = torch.full((bt, n), 1.0, dtype=torch.float16, device=dev)
    bsa.gemm_packed(xt, packed, n, to_dev(want.astype(np.int32), dev), y_list, num_active=c, plan=pl,
                    workspace_prefix="t_self_nonfinite")
    torch.cuda.synchronize()
    assert torch.equal(torch.isnan(y), torch.isnan(y_list)) and torch.equal(torch.isinf(y), torch.isinf(y_list))
    assert bool(torch.isnan(y[nan_row]).all())
    finite_rows = [r for r in range(bt) if r not in (inf_row, nan_row)]
    if finite_rows:
        assert torch.equal(y[finite_rows], y_list[finite_rows])
        assert_close(y[finite_rows].float().cpu().numpy(), orc.gemm_ref(x[finite_rows], w_nk, want),
                     f"finite rows bt={bt} K={kdim}")


def test_two_launch_selection_above_the_self_scoring_size(dev):
    """Above 24 KiB of activations (bt x K x 2) or 8 rows, and on the dot-product kernel (kind 3),
    the score launch runs, writing the block scores into the selector's part of the workspace."""
    import ctypes

    from bsa_mi355x import _lib
    from bsa_mi355x.runtime import _stream_handle

    lib = bsa.load()
    for bt, kdim, plan in ((16, 4096, (1, 16, 4, 4, 16, 1)), (4, 11008, (1, 16, 4, 4, 16, 1)),
                           (4, 4096, (1, 16, 4, 4, 16, 6)), (2, 4096, (1, 16, 4, 4, 2, 3))):
        n, k = 512, 20
        x, w_nk, _ = case(950 + bt, bt, kdim, n, 1, "normal")
        xt = to_dev(x, dev)
        packed = bsa.pack_weight(to_dev(w_nk, dev))
        pl = bsa.Plan(*plan)
        sel = int(lib.bsg_select_workspace_bytes(kdim))
        ws = torch.zeros(sel + int(lib.bsg_gemm_workspace_bytes(bt, n, ctypes.byref(pl))), dtype=torch.uint8,
                         device=dev)
        ws[256:sel] = 0xAB
        y = torch.empty(bt, n, dtype=torch.float16, device=dev)
        idx = torch.empty(k, dtype=torch.int32, device=dev)
        cnt = torch.empty(1, dtype=torch.int32, device=dev)
        rc = lib.bsg_select_gemm(xt.data_ptr(), kdim, bt, kdim, k, packed.data_ptr(), n, idx.data_ptr(),
                                 cnt.data_ptr(), y.data_ptr(), n, 0, ws.data_ptr(), ws.numel(), ctypes.byref(pl),
                                 _stream_handle(dev))
        assert rc == _lib.BSG_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert not bool((ws[256:sel] == 0xAB).all()), f"bt={bt} K={kdim}: no score launch"
        want = orc.select_topk_l1(x, k)
        assert np.array_equal(idx.cpu().numpy(), want)
        assert_close(y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), f"two-launch bt={bt} K={kdim}")


def test_select_density_wrapper(dev):
    x = np.random.default_rng(9).normal(0, 1, size=(64, 4096)).astype(np.float16)
    got = bsa._select_active_blocks_l1(to_dev(x, dev).view(64, 1, 4096), 0.48)
    torch.cuda.synchronize()
    assert got.dtype == torch.int32 and got.numel() == orc.n_keep(0.48, 64) == 31
    assert np.array_equal(got.cpu().numpy(), orc.select_topk_l1(x, 31))


# ---------------------------------------------------------------------------------------
# Reference scoring rules (L2 mean, energy, prior, channel scale, energy budget), fp64 scores:
# the kept set and count must equal the float64 oracle's; the kept-energy ratio within 1e-6.


def _scored(dev, x, k, dtype=torch.float16, **kw):
    kw = {n: (to_dev(np.asarray(v, np.float32), dev, torch.float32) if isinstance(v, np.ndarray) else v)
          for n, v in kw.items()}
    xt = torch.from_numpy(np.asarray(x, np.float32)).to(dtype).to(dev)
    ratio = torch.empty(1, dtype=torch.float32, device=dev)
    idx, cnt, _ = bsa.select_topk(xt, k, ratio_out=ratio, **kw)
    torch.cuda.synchronize()
    c = int(cnt.item())
    return idx[:c].cpu().numpy(), c, float(ratio.item())


@pytest.mark.parametrize("score,prior,scale,keep", [("l2_mean", False, False, 0.0), ("energy", False, False, 0.0),
                                                    ("energy", False, True, 0.0), ("l2_mean", True, False, 0.0),
                                                    ("energy", True, False, 0.9), ("l2_mean", False, False, 0.75)])
@pytest.mark.parametrize("bt,kdim,k", [(1, 4096, 13), (16, 4096, 23), (64, 4096, 31), (64, 11008, 83),
                                       (5, 1000, 4), (33, 2048, 1)])
def test_scored_selector_matches_oracle(dev, score, prior, scale, keep, bt, kdim, k):
    rng = np.random.default_rng(bt * 13 + k)
    x = rng.laplace(0, 0.05, size=(bt, kdim)).astype(np.float16)
    nb = kdim // 64
    kw = dict(score=score, energy_keep=keep)
    if prior:
        kw.update(block_prior=rng.uniform(0, 1, size=nb).astype(np.float32), prior_alpha=0.7, prior_eps=0.1)
    if scale:
        kw["channel_scale"] = rng.uniform(0.5, 2, size=kdim).astype(np.float32)
    got, cnt, ratio = _scored(dev, x, k, **kw)
    want, wkeep, wratio = orc.select_scored_ref(x, k, score, prior=kw.get("block_prior"), alpha=0.7, eps=0.1,
                                                scale=kw.get("channel_scale"), energy_keep=keep)
    assert cnt == wkeep and np.array_equal(got, want), (cnt, wkeep)
    assert abs(ratio - wratio) <= 1e-6 * max(wratio, 1e-12) + 1e-7


def test_scored_selector_bf16_and_closed_form_budget(dev):
    x = np.zeros((3, 5 * 64), dtype=np.float32)
    for j, m in enumerate((32, 16, 8, 4, 4)):
        x[:, 64 * j:64 * j + m] = 1.0
    for dt in (torch.float16, torch.bfloat16):
        got, cnt, ratio = _scored(dev, x, 1, dtype=dt, score="energy", energy_keep=0.8)
        assert cnt == 3 and np.array_equal(got, [0, 1, 2]) and ratio == 56 / 64
    rng = np.random.default_rng(9)
    xb = rng.normal(0, 1, size=(16, 4096)).astype(np.float32)
    xb16 = torch.from_numpy(xb).to(torch.bfloat16).float().numpy()  # the values the kernel sees
    got, cnt, _ = _scored(dev, xb, 20, dtype=torch.bfloat16, score="l2_mean")
    want, _, _ = orc.select_scored_ref(xb16, 20, "l2_mean")
    assert np.array_equal(got, want)


def test_reference_selector_drop_ins(dev):
    """_select_active_blocks / _topk_energy_ratio / _energy_expanded_active_blocks keep the
    reference's signatures (RRD:90-176) and agree with the oracle."""
    rng = np.random.default_rng(11)
    x = rng.laplace(0, 0.05, size=(16, 11008)).astype(np.float16)
    x3 = to_dev(x, dev).view(16, 1, 11008)
    idx = bsa._select_active_blocks(x3, 0.36, 64)
    want, _, _ = orc.select_scored_ref(x, orc.n_keep(0.36, 172), "l2_mean")
    assert np.array_equal(idx.cpu().numpy(), want)
    r = bsa._topk_energy_ratio(x3, 0.36, 64)
    _, _, wr = orc.select_scored_ref(x, orc.n_keep(0.36, 172), "energy")
    assert abs(r - wr) < 1e-6
    active, ratio, dens = bsa._energy_expanded_active_blocks(x3, 0.2, 64, 0.5)
    want, keep, wr = orc.select_scored_ref(x, orc.n_keep(0.2, 172), "energy", energy_keep=0.5)
    assert np.array_equal(active.cpu().numpy(), want) and abs(ratio - wr) < 1e-6 and dens == keep / 172
    assert bsa._energy_expanded_active_blocks(x3, 1.0, 64, 0.5) == (None, 1.0, 1.0)


def test_budget_selection_feeds_gemm_by_device_count(dev):
    """The budget selector's device-side count drives the GEMM without a host round trip."""
    bt, k, n = 16, 4096, 1024
    x, w_nk, _ = case(41, bt, k, n, 1)
    xt = to_dev(x, dev)
    idx, cnt, _ = bsa.select_topk(xt, 8, score="energy", energy_keep=0.6)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    out = torch.empty(bt, n, dtype=torch.float16, device=dev)
    bsa.gemm_packed(xt, packed, n, idx, out, num_active=idx.numel(), num_active_dev=cnt)
    torch.cuda.synchronize()
    c = int(cnt.item())
    want, keep, _ = orc.select_scored_ref(x, 8, "energy", energy_keep=0.6)
    assert c == keep and np.array_equal(idx[:c].cpu().numpy(), want)
    assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, want), "budget selection -> GEMM")


def test_reference_drop_ins_ignore_a_prior_of_the_wrong_length(dev):
    """The reference applies block_prior only when it has floor(K/64) entries and ignores it
    otherwise (RRD:110-112, 135-138, 161-164): a shorter or longer prior gives the no-prior
    result in all three drop-ins; the matching-length prior changes the selection; the library
    entry point itself rejects a wrong length."""
    rng = np.random.default_rng(12)
    x = rng.laplace(0, 0.05, size=(16, 4096)).astype(np.float16)
    x3 = to_dev(x, dev).view(16, 1, 4096)
    base = bsa._select_active_blocks(x3, 0.3, 64).cpu().numpy()
    r0 = bsa._topk_energy_ratio(x3, 0.3, 64)
    e0, er0, ed0 = bsa._energy_expanded_active_blocks(x3, 0.2, 64, 0.5)
    for length in (63, 65):
        prior = torch.linspace(0.0, 3.0, length, device=dev)
        assert np.array_equal(bsa._select_active_blocks(x3, 0.3, 64, block_prior=prior).cpu().numpy(), base)
        assert bsa._topk_energy_ratio(x3, 0.3, 64, block_prior=prior) == r0
        e, er, ed = bsa._energy_expanded_active_blocks(x3, 0.2, 64, 0.5, block_prior=prior)
        assert np.array_equal(e.cpu().numpy(), e0.cpu().numpy()) and er == er0 and ed == ed0
        with pytest.raises(ValueError):
            bsa.select_topk(x3, 19, score="l2_mean", block_prior=prior)
    prior = torch.linspace(0.0, 3.0, 64, device=dev)
    got = bsa._select_active_blocks(x3, 0.3, 64, block_prior=prior).cpu().numpy()
    want, _, _ = orc.select_scored_ref(x, orc.n_keep(0.3, 64), "l2_mean", prior=prior.cpu().numpy())
    assert np.array_equal(got, want) and not np.array_equal(got, base)



# ---------------------------------------------------------------------------------------
# Selection by the reference's rules + GEMM in one library call (bsg_select_gemm_rule): the
# kept ids, count and ratio must be select_topk's (and the float64 oracle's) for the same x and
# options, and Y the GEMM on that list.


def _rule_call(dev, x, w_nk, k, dtype=torch.float16, plan=None, **kw):
    from bsa_mi355x.select import select_gemm_rule_packed

    kw = {n: (to_dev(np.asarray(v, np.float32), dev, torch.float32) if isinstance(v, np.ndarray) else v)
          for n, v in kw.items()}
    bt, kdim = x.shape
    n = w_nk.shape[0]
    xt = torch.from_numpy(np.asarray(x, np.float32)).to(dtype).to(dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev, dtype))
    y = torch.full((bt, n), float("nan"), dtype=dtype, device=dev)
    print(f"rule select+gemm bt={bt} K={kdim} N={n} k={k} {dtype} plan={plan} opts={sorted(kw)}", flush=True)
    idx, cnt, ratio = select_gemm_rule_packed(xt, packed, n, k, y, plan=plan, **kw)
    torch.cuda.synchronize()
    c = int(cnt.item())
    sel_idx, sel_cnt, sel_ratio = bsa.select_topk(xt, k, **kw)
    torch.cuda.synchronize()
    return (idx[:c].cpu().numpy(), c, None if ratio is None else float(ratio.item()), y, xt, packed,
            (sel_idx[:int(sel_cnt.item())].cpu().numpy(), int(sel_cnt.item()),
             None if sel_ratio is None else float(sel_ratio.item())))


@pytest.mark.parametrize("bt,kdim,n,k", [(16, 4096, 4096, 23), (64, 4096, 11008, 31), (64, 11008, 4096, 83)])
@pytest.mark.parametrize("score,prior,scale", [("l2_mean", False, False), ("l2_mean", True, False),
                                               ("energy", False, True), ("energy", True, False)])
def test_rule_select_gemm_matches_selector_and_oracle(dev, bt, kdim, n, k, score, prior, scale):
    """The reference's decode linear (select -> GEMM, RRD:179-284) as one call at the shapes of
    BASELINE's batches: ids and count equal the oracle's (select_scored_ref) and the separate
    selector's; Y is within tolerance of gemm_ref on those blocks and bit for bit the GEMM on
    the same list with the same plan."""
    rng = np.random.default_rng(bt * 7 + k)
    x = rng.laplace(0, 0.05, size=(bt, kdim)).astype(np.float16)
    w_nk = (rng.normal(0, 0.02, size=(n, kdim))).astype(np.float16)
    nb = kdim // 64
    kw = dict(score=score)
    if prior:
        kw.update(block_prior=rng.uniform(0, 1, size=nb).astype(np.float32), prior_alpha=0.7, prior_eps=0.1)
    if scale:
        kw["channel_scale"] = rng.uniform(0.5, 2, size=kdim).astype(np.float32)
    got, c, _, y, xt, packed, (s_idx, s_cnt, _) = _rule_call(dev, x, w_nk, k, **kw)
    want, keep, _ = orc.select_scored_ref(x, k, score, prior=kw.get("block_prior"), alpha=0.7, eps=0.1,
                                          scale=kw.get("channel_scale"))
    assert c == keep == min(k, nb) and np.array_equal(got, want)
    assert s_cnt == c and np.array_equal(s_idx, want)
    assert_close(y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), f"rule {score} bt={bt} K={kdim}")
    pl = bsa.resolve_plan(bt, n, -(-kdim // 64), min(k, nb), dev, None, select=True)
    y_list = torch.full_like(y, float("nan"))
    bsa.gemm_packed(xt, packed, n, to_dev(want.astype(np.int32), dev), y_list, num_active=c, plan=pl,
                    workspace_prefix="t_rule_ref")
    torch.cuda.synchronize()
    assert torch.equal(y, y_list)


def test_rule_select_gemm_three_launch_forms_and_edges(dev):
    """The forms that rank in a separate launch (an energy budget with its ratio, bf16, a
    dot-product plan) give the selector's ids, count and ratio too; a partial last K-block is
    never kept (floor(K/64) scored blocks), k above the block count keeps every scored block,
    k = 0 writes zeros, and negative scores (a negative channel scale) rank below the rest."""
    rng = np.random.default_rng(5)
    # energy budget + ratio: three launches, the GEMM on the device count
    x = rng.laplace(0, 0.05, size=(16, 4096)).astype(np.float16)
    w_nk = rng.normal(0, 0.02, size=(1024, 4096)).astype(np.float16)
    got, c, ratio, y, _, _, (s_idx, s_cnt, s_ratio) = _rule_call(dev, x, w_nk, 8, score="energy", energy_keep=0.6)
    want, keep, wratio = orc.select_scored_ref(x, 8, "energy", energy_keep=0.6)
    assert c == keep == s_cnt and keep > 8 and np.array_equal(got, want) and np.array_equal(s_idx, want)
    assert ratio == s_ratio and abs(ratio - wratio) <= 1e-6
    assert_close(y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), "energy budget")
    # bf16
    xb = rng.normal(0, 1, size=(16, 4096)).astype(np.float32)
    xb16 = torch.from_numpy(xb).to(torch.bfloat16).float().numpy()
    wb = rng.normal(0, 0.02, size=(512, 4096)).astype(np.float32)
    wb16 = torch.from_numpy(wb).to(torch.bfloat16).float().numpy()
    got, c, _, y, _, _, (s_idx, _, _) = _rule_call(dev, xb, wb, 20, dtype=torch.bfloat16, score="l2_mean")
    want, _, _ = orc.select_scored_ref(xb16, 20, "l2_mean")
    assert c == 20 and np.array_equal(got, want) and np.array_equal(s_idx, want)
    ref = orc.gemm_ref(xb16.astype(np.float32), wb16.astype(np.float32), want)
    yb = y.float().cpu().numpy()
    assert orc.rel_frobenius(yb, ref) <= 5e-3
    # a dot-product (kind 3) plan at 4 rows: no selection instantiation, rank launch
    x4 = rng.laplace(0, 0.05, size=(4, 4096)).astype(np.float16)
    got, c, _, y, _, _, (s_idx, _, _) = _rule_call(dev, x4, w_nk, 13, plan=bsa.Plan(1, 16, 4, 4, 4, 3),
                                                   score="l2_mean")
    want, _, _ = orc.select_scored_ref(x4, 13, "l2_mean")
    assert c == 13 and np.array_equal(got, want) and np.array_equal(s_idx, want)
    assert_close(y.float().cpu().numpy(), orc.gemm_ref(x4, w_nk, want), "kind 3 plan")
    # K tail: 15 scored blocks of 16; k past them keeps the 15 scored blocks only
    xt_ = rng.laplace(0, 0.05, size=(16, 1000)).astype(np.float16)
    xt_[:, 960:] = 30.0  # the partial block would win if it were scored
    wt_ = rng.normal(0, 0.02, size=(256, 1000)).astype(np.float16)
    got, c, _, y, _, _, _ = _rule_call(dev, xt_, wt_, 40, score="l2_mean")
    assert c == 15 and np.array_equal(got, np.arange(15))
    assert_close(y.float().cpu().numpy(), orc.gemm_ref(xt_, wt_, np.arange(15)), "K tail")
    got, c, _, y, _, _, _ = _rule_call(dev, xt_, wt_, 6, score="energy")
    want, _, _ = orc.select_scored_ref(xt_, 6, "energy")
    assert c == 6 and np.array_equal(got, want) and 15 not in got
    # k = 0: nothing kept, zeros
    got, c, _, y, _, _, _ = _rule_call(dev, x, w_nk, 0, score="l2_mean")
    assert c == 0 and torch.count_nonzero(y).item() == 0
    # negative channel scale: odd blocks score below zero
    scale = np.where(np.arange(4096) // 64 % 2 == 0, 1.0, -1.0).astype(np.float32)
    for k in (20, 40):
        got, c, _, y, _, _, (s_idx, _, _) = _rule_call(dev, x, w_nk, k, score="energy", channel_scale=scale)
        want, _, _ = orc.select_scored_ref(x, k, "energy", scale=scale)
        assert c == k and np.array_equal(got, want) and np.array_equal(s_idx, want), k
        assert_close(y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), f"negative scale k={k}")


def test_rule_select_gemm_ranks_a_nan_block_first(dev):
    """A NaN activation makes its block's score NaN, which ranks above every number (as
    torch.topk ranks NaN); ties between equal scores still go to the lower block id."""
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, size=(16, 4096)).astype(np.float16)
    x[3, 64 * 40 + 9] = np.float16(np.nan)
    for j in (10, 20, 30):
        x[:, 64 * j:64 * j + 64] = 40.0
    w_nk = rng.normal(0, 0.02, size=(512, 4096)).astype(np.float16)
    for score in ("l2_mean", "energy"):
        got, c, _, _, _, _, (s_idx, _, _) = _rule_call(dev, x, w_nk, 3, score=score)
        want, _, _ = orc.select_scored_ref(x, 3, score)
        assert c == 3 and np.array_equal(got, [10, 20, 40]) and np.array_equal(want, [10, 20, 40])
        assert np.array_equal(s_idx, want)
