"""GPU parity of the 2-D block-sparse path (active K-blocks and active 64-column output
blocks), its compact output, the scatter back to dense and the mask -> block list."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from bsa_mi355x import sparse2d as s2d
from helpers import assert_close, case, to_dev
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu

SENTINEL = 7.0  # columns a 2-D launch must not touch keep this value, bit for bit


def _run(dev, x, w_nk, kb, nb, compact, plan=None, num_n_dev=None, num_n=None):
    bt, _ = x.shape
    n = w_nk.shape[0]
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    nn = len(nb) if num_n is None else num_n
    width = 64 * nn if compact else n
    y = torch.full((bt, width), SENTINEL, dtype=torch.float16, device=dev)
    s2d.gemm_2d_packed(to_dev(x, dev), packed, n, None if kb is None else to_dev(np.asarray(kb, np.int32), dev),
                       to_dev(np.asarray(nb, np.int32), dev), y, compact=compact, num_n=num_n,
                       num_n_dev=num_n_dev, plan=None if plan is None else bsa.Plan(*plan))
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


def _check(y, x, w_nk, kb, nb, compact, what):
    kb_ref = np.arange(orc.nblk_of(x.shape[1])) if kb is None else kb
    init = np.full((x.shape[0], w_nk.shape[0]), SENTINEL, dtype=np.float32)
    want = orc.gemm_2d_ref(x, w_nk, kb_ref, nb, out_init=init, compact=compact)
    if compact:
        assert_close(y, want, what)
    else:
        n = w_nk.shape[0]
        written = np.zeros(n, bool)
        for b in nb:
            if 0 <= b < (n + 63) // 64:
                written[64 * b:min(64 * b + 64, n)] = True
        assert np.all(y[:, ~written] == SENTINEL), f"{what}: columns outside the active blocks were written"
        if written.any():
            assert_close(y[:, written], want[:, written], what)


@pytest.mark.parametrize("bt,kdim,n,na,nb,plan", [
    (16, 4096, 4096, 23, [0, 5, 6, 63], (1, 16, 2, 4, 16, 1)),   # waves split the list
    (16, 11008, 4096, 62, [3, 9, 40], (4, 16, 4, 4, 16, 1)),      # split-K 4
    (64, 4096, 11008, 31, [1, 2, 3, 100, 171], (1, 16, 8, 4, 64, 4)),  # channel-half waves
    (32, 4096, 4096, 20, [10, 11], (2, 16, 4, 4, 32, 2)),         # X tile in LDS, split-K 2
    (2, 4096, 1000, 13, [0, 15], (1, 16, 4, 4, 2, 3)),            # dot-product kernel, partial last block
    (5, 1000, 4000, 6, [0, 62], None),                            # odd sizes, automatic plan
])
@pytest.mark.parametrize("compact", [False, True])
def test_2d_matches_oracle(dev, bt, kdim, n, na, nb, plan, compact):
    x, w_nk, kb = case(51 + bt, bt, kdim, n, na, "normal")
    y = _run(dev, x, w_nk, kb, nb, compact, plan)
    _check(y, x, w_nk, kb, nb, compact, f"2d bt={bt} K={kdim} N={n} plan={plan} compact={compact}")


def test_2d_dense_k_and_every_block_equals_1d(dev):
    """Every output block listed (dense K) gives exactly the 1-D kernel's result."""
    bt, kdim, n = 16, 4096, 4096
    x, w_nk, _ = case(61, bt, kdim, n, 1, "normal")
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    xt = to_dev(x, dev)
    y1 = torch.empty(bt, n, dtype=torch.float16, device=dev)
    pl = bsa.Plan(1, 16, 2, 4, 16, 1)
    bsa.gemm_packed(xt, packed, n, None, y1, plan=pl)
    y2 = torch.empty(bt, n, dtype=torch.float16, device=dev)
    s2d.gemm_2d_packed(xt, packed, n, None, torch.arange(64, dtype=torch.int32, device=dev), y2, plan=pl)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_2d_invalid_ids_and_device_count(dev):
    bt, kdim, n = 16, 4096, 1000  # 16 output blocks, the last one partial
    x, w_nk, kb = case(62, bt, kdim, n, 20, "normal")
    nb = [2, -1, 16, 5]  # two ids outside [0, 16)
    _check(_run(dev, x, w_nk, kb, nb, False), x, w_nk, kb, nb, False, "invalid ids in place")
    _check(_run(dev, x, w_nk, kb, nb, True), x, w_nk, kb, nb, True, "invalid ids compact")
    # a device count of 2 leaves list entries 2.. unwritten
    cnt = torch.tensor([2], dtype=torch.int32, device=dev)
    y = _run(dev, x, w_nk, kb, [1, 3, 7, 9], False, num_n_dev=cnt)
    _check(y, x, w_nk, kb, [1, 3], False, "device count")


def test_compact_scatter_is_in_place_result(dev):
    bt, kdim, n = 8, 4096, 4096
    x, w_nk, kb = case(63, bt, kdim, n, 30, "normal")
    nb = [0, 7, 8, 33, 63]
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    xt, kbt, nbt = to_dev(x, dev), to_dev(kb, dev), to_dev(np.asarray(nb, np.int32), dev)
    yin = torch.full((bt, n), SENTINEL, dtype=torch.float16, device=dev)
    s2d.gemm_2d_packed(xt, packed, n, kbt, nbt, yin)
    comp = torch.empty(bt, 64 * len(nb), dtype=torch.float16, device=dev)
    s2d.gemm_2d_packed(xt, packed, n, kbt, nbt, comp, compact=True)
    ysc = torch.full((bt, n), SENTINEL, dtype=torch.float16, device=dev)
    s2d.scatter_nblocks(comp, nbt, ysc)
    torch.cuda.synchronize()
    assert torch.equal(yin, ysc)


@pytest.mark.parametrize("n,p", [(64, 0.5), (1000, 0.01), (11008, 0.002), (4096, 0.0), (130, 1.0)])
def test_nmask_blocks(dev, n, p):
    m = (np.random.default_rng(n).random(n) < p).astype(np.uint8)
    blocks, cnt = s2d.nmask_blocks(to_dev(m, dev))
    torch.cuda.synchronize()
    want = orc.nmask_blocks_ref(m, n)
    c = int(cnt.item())
    assert c == len(want)
    assert np.array_equal(blocks.cpu().numpy()[:c], want)
    assert np.array_equal(s2d._get_cached_active_n_blocks_delta(to_dev(m, dev), "t", 64).cpu().numpy(), want)


def test_reference_2d_entry_points(dev):
    """The reference's 2-D names and return values: in place, zero fill, compact + scatter,
    a mask-driven output list, the compact wrapper and the empty cases."""
    bsz, kdim, n = 4, 4096, 4096
    x, w_nk, kb = case(64, bsz, kdim, n, 25, "normal")
    x3 = to_dev(x, dev).view(bsz, 1, kdim)
    w = to_dev(w_nk, dev)
    kbt = to_dev(kb[::-1].copy(), dev)  # unsorted: the wrapper sorts
    nb = np.array([40, 3, 12], dtype=np.int32)
    out = torch.full((bsz, 1, n), SENTINEL, dtype=torch.float16, device=dev)
    c, blocks = s2d._prepacked_block_sparse_gemm_2d_from_active_blocks(x3, w, kbt, to_dev(nb, dev), out)
    assert c is None and np.array_equal(blocks.cpu().numpy(), np.sort(nb))
    _check(out.view(bsz, n).float().cpu().numpy(), x, w_nk, kb, np.sort(nb), False, "reference in place")
    out.fill_(SENTINEL)
    s2d._prepacked_block_sparse_gemm_2d_from_active_blocks(x3, w, kbt, to_dev(nb, dev), out, zero_fill_out=True)
    want = orc.gemm_2d_ref(x, w_nk, kb, nb, out_init=np.zeros((bsz, n)))
    assert_close(out.view(bsz, n).float().cpu().numpy(), want, "zero fill")
    out.fill_(SENTINEL)
    c, blocks = s2d._prepacked_block_sparse_gemm_2d_from_active_blocks(
        x3, w, kbt, to_dev(nb, dev), out, compact_output=True, scatter_compact_to_dense=True, zero_fill_out=True)
    assert c.shape == (bsz, 1, 192)
    assert_close(c.view(bsz, 192).float().cpu().numpy(), orc.gemm_2d_ref(x, w_nk, kb, np.sort(nb), compact=True),
                 "reference compact")
    assert_close(out.view(bsz, n).float().cpu().numpy(), want, "reference compact + scatter")
    mask = np.zeros(n, np.uint8)
    mask[[5, 700, 701, 4095]] = 1  # blocks 0, 10, 63
    out.fill_(SENTINEL)
    _, blocks = s2d._prepacked_block_sparse_gemm_2d_from_active_blocks(
        x3, w, kbt, None, out, active_n_mask_u8=to_dev(mask, dev))
    assert np.array_equal(blocks.cpu().numpy(), [0, 10, 63])
    _check(out.view(bsz, n).float().cpu().numpy(), x, w_nk, kb, [0, 10, 63], False, "mask-driven")
    comp, blocks = s2d._prepacked_block_sparse_gemm_2d_compact_from_active_blocks(x3, w, kbt, to_dev(nb, dev))
    assert comp.shape == (bsz, 1, 192)
    assert_close(comp.view(bsz, 192).float().cpu().numpy(),
                 orc.gemm_2d_ref(x, w_nk, kb, np.sort(nb), compact=True), "compact wrapper")
    empty, eb = s2d._prepacked_block_sparse_gemm_2d_compact_from_active_blocks(x3, w, kbt, None)
    assert empty.shape == (bsz, 1, 0) and eb.numel() == 0
    out.fill_(SENTINEL)
    c, eb = s2d._prepacked_block_sparse_gemm_2d_from_active_blocks(
        x3, w, kbt[:0], to_dev(nb, dev), out)
    assert c is None and eb.numel() == 0 and not torch.any(out)


def test_2d_rejects_a_wide_plan(dev):
    bt, kdim, n = 32, 4096, 4096
    x, w_nk, kb = case(65, bt, kdim, n, 10, "normal")
    with pytest.raises(ValueError):
        _run(dev, x, w_nk, kb, [1], False, plan=(1, 32, 4, 4, 32, 2))  # 128 columns per work-group
    with pytest.raises(ValueError):
        _run(dev, x, w_nk, kb, [1], False, plan=(1, 48, 2, 4, 32, 6))  # variable-width groups: no 2-D kernel


@pytest.mark.parametrize("bt,na", [(4, 6), (4, 25), (16, 23), (64, 31)])
def test_2d_auto_plan_when_the_tuned_1d_plan_is_variable_width(dev, bt, na):
    """The automatic 2-D plan starts from the tuned 1-D plan of the same problem; where that is a
    variable-width kind (5/6, no 2-D instantiation) it takes the 16-column list-splitting tile
    of the same rows instead, with its own split-K, and matches the oracle."""
    from bsa_mi355x import sparse2d as s2d_mod

    kdim, n = 4096, 4096
    x, w_nk, kb = case(90 + bt, bt, kdim, n, na, "normal")
    pl = s2d_mod.plan_2d(bt, n, 3, orc.nblk_of(kdim), na, dev)
    assert pl.kind in (1, 2, 3, 4) and pl.group_cols() <= 64, pl
    _check(_run(dev, x, w_nk, kb, [0, 17, 63], False), x, w_nk, kb, [0, 17, 63], False, f"auto 2-D B={bt} na={na}")


def test_every_2d_tile(dev):
    """Every tile with a 2-D instantiation (work-group columns dividing 64): fp16 in place and
    compact, and bf16 in place, over output blocks that include the partial last one.  Columns
    outside the listed blocks keep the sentinel bit for bit."""
    bt, kdim, n = 37, 4096, 1000  # 16 output blocks, the last 40 columns wide; 3 row groups of 16
    x, w_nk, kb = case(66, bt, kdim, n, 29, "normal")
    nb = [0, 3, 15]
    xb = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    wb = torch.from_numpy(w_nk.astype(np.float32)).to(torch.bfloat16)
    init = np.full((bt, n), SENTINEL, dtype=np.float32)
    ref = {c: orc.gemm_2d_ref(x, w_nk, kb, nb, out_init=init, compact=c) for c in (False, True)}
    ref_b = orc.gemm_2d_ref(xb.float().numpy(), wb.float().numpy(), kb, nb, out_init=init)
    written = np.zeros(n, bool)
    for b in nb:
        written[64 * b:min(64 * b + 64, n)] = True
    packed, packed_b = bsa.pack_weight(to_dev(w_nk, dev)), bsa.pack_weight(wb.to(dev))
    xt, xbt = to_dev(x, dev), xb.to(dev)
    kbt, nbt = to_dev(kb, dev), to_dev(np.asarray(nb, np.int32), dev)
    tiles = [t for t in bsa.kernel_tiles()
             if 64 % bsa.Plan(1, t[2], t[3], t[4], t[1], t[0]).group_cols() == 0]
    assert len(tiles) >= 50
    for kind, rows, cols, waves, depth in tiles:
        p = bsa.Plan(1 if kind == 3 else 2, cols, waves, depth, rows, kind)
        what = f"2d tile kind={kind} rows={rows} cols={cols} waves={waves} depth={depth}"
        print(what, flush=True)
        for compact in (False, True):
            y = torch.full((bt, 64 * len(nb) if compact else n), SENTINEL, dtype=torch.float16, device=dev)
            s2d.gemm_2d_packed(xt, packed, n, kbt, nbt, y, compact=compact, plan=p)
            torch.cuda.synchronize()
            yv = y.float().cpu().numpy()
            if compact:
                assert_close(yv, ref[True], f"{what} compact")
            else:
                assert np.all(yv[:, ~written] == SENTINEL), f"{what}: columns outside the blocks were written"
                assert_close(yv[:, written], ref[False][:, written], what)
        yb = torch.full((bt, n), SENTINEL, dtype=torch.bfloat16, device=dev)
        s2d.gemm_2d_packed(xbt, packed_b, n, kbt, nbt, yb, plan=p)
        torch.cuda.synchronize()
        ybv = yb.float().cpu().numpy()
        assert np.all(ybv[:, ~written] == SENTINEL), f"{what} bf16: columns outside the blocks were written"
        # bf16 output keeps 8 significant bits: tolerance 5e-3 rel. Frobenius, 2e-2 max-abs
        got, want = ybv[:, written], ref_b[:, written]
        rf = orc.rel_frobenius(got, want)
        assert rf <= 5e-3 and np.max(np.abs(got - want)) <= 2e-2 * np.max(np.abs(want)), f"{what} bf16: {rf:.3e}"


def test_2d_split_k_workspace_reuse_across_block_counts(dev):
    """One cached workspace serves split-K 2-D launches with different active output-block
    counts: the arrival counters sit at a fixed offset whatever a launch's tile count, so a
    launch over many blocks after one over few (and a few-block launch again) is exact."""
    bt, kdim, n = 16, 4096, 4096
    x, w_nk, kb = case(64, bt, kdim, n, 40, "normal")
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    xt, kbt = to_dev(x, dev), to_dev(kb, dev)
    plan = bsa.Plan(4, 16, 4, 4, 16, 1)  # split-K 4, 16-column work-groups: 4 tiles per output block
    rng = np.random.default_rng(5)
    for nn in (3, 20, 64, 3, 20):
        nb = np.sort(rng.choice(64, nn, replace=False)).astype(np.int32)
        y = torch.full((bt, n), SENTINEL, dtype=torch.float16, device=dev)
        pl = s2d.gemm_2d_packed(xt, packed, n, kbt, to_dev(nb, dev), y, plan=plan, workspace_prefix="ws_reuse_2d")
        assert pl.split_k == 4
        torch.cuda.synchronize()
        _check(y.float().cpu().numpy(), x, w_nk, kb, nb, False, f"workspace reuse nn={nn}")
