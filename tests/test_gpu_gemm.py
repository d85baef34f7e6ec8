"""GPU parity of the block-sparse GEMM (HIP, gfx950) against the CPU oracle.

Bar (BASELINE): relative Frobenius error <= 1e-3 and max-abs error <= 1e-2 * max|Y_ref| for
fp16 inputs with fp32 accumulation; the reference is oracle.bsg_oracle.gemm_ref64 (gather +
matmul in float64) or gemm_ref (float32, BASELINE's CPU path) at full Llama sizes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bsa_mi355x as bsa
from helpers import assert_close, case, to_dev
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu

F16 = torch.float16


def _run_list(dev, x, w_nk, idx, plan=None, prefix="t", sort=True, dtype=F16):
    bt, k = x.shape
    n = w_nk.shape[0]
    xt = to_dev(x, dev, dtype).view(bt, 1, k)
    wt = to_dev(w_nk, dev, dtype)
    it = to_dev(np.asarray(idx, dtype=np.int32), dev)
    out = torch.full((bt, 1, n), float("nan"), dtype=dtype, device=dev)
    if plan is None:
        bsa._prepacked_block_sparse_gemm_from_active_blocks(xt, wt, it, out, cache_prefix=prefix,
                                                            sort_active_blocks=sort)
    else:
        bsa._prepacked_block_sparse_gemm_from_active_blocks_splitk(xt, wt, it, out, cache_prefix=prefix, **plan)
    torch.cuda.synchronize()
    return out.view(bt, n).float().cpu().numpy()


@pytest.mark.parametrize("bt,k,n,na", [
    (1, 64, 16, 1),
    (2, 128, 32, 1),
    (3, 256, 48, 2),
    (16, 1024, 256, 8),
    (17, 512, 100, 5),      # N not a multiple of 16, bt not a multiple of 16
    (33, 2048, 520, 13),
    (64, 4096, 1024, 31),
    (100, 1024, 384, 9),    # bt above 64 rows: more grid rows
])
def test_small_shapes(dev, bt, k, n, na):
    x, w_nk, idx = case(100 + bt, bt, k, n, na)
    y = _run_list(dev, x, w_nk, idx, prefix=f"small{bt}")
    assert_close(y, orc.gemm_ref64(x, w_nk, idx), f"bt={bt} k={k} n={n} na={na}")


def test_k_tail_block(dev):
    """K not a multiple of 64: the last block is partial (reference masks rk < M, KRN:709-717)."""
    bt, k, n = 5, 1000, 64
    nb = orc.nblk_of(k)
    x, w_nk, _ = case(7, bt, k, n, 1)
    idx = np.array([0, 3, nb - 1], dtype=np.int32)
    assert_close(_run_list(dev, x, w_nk, idx, prefix="ktail"), orc.gemm_ref64(x, w_nk, idx), "k tail")


def test_k_not_multiple_of_8(dev):
    bt, k, n = 3, 203, 32
    x, w_nk, _ = case(8, bt, k, n, 1)
    idx = np.array([1, 3], dtype=np.int32)
    assert_close(_run_list(dev, x, w_nk, idx, prefix="k203"), orc.gemm_ref64(x, w_nk, idx), "k=203")


def test_zero_active_writes_zeros(dev):
    x, w_nk, _ = case(9, 4, 256, 64, 1)
    xt = to_dev(x, dev).view(4, 1, 256)
    wt = to_dev(w_nk, dev)
    out = torch.full((4, 1, 64), 7.0, dtype=F16, device=dev)
    bsa._prepacked_block_sparse_gemm_from_active_blocks(xt, wt, torch.empty(0, dtype=torch.int32, device=dev), out)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


def test_out_of_range_ids_contribute_nothing(dev):
    bt, k, n = 4, 512, 64
    x, w_nk, _ = case(10, bt, k, n, 1)
    idx = np.array([1, 8, 5, 1000, -3], dtype=np.int32)  # nblk = 8: ids 8, 1000, -3 are outside
    y = _run_list(dev, x, w_nk, idx, prefix="oor", sort=False)
    assert_close(y, orc.gemm_ref64(x, w_nk, [1, 5]), "out-of-range ids")


def test_unsorted_list_and_limit(dev):
    bt, k, n = 8, 1024, 128
    x, w_nk, _ = case(11, bt, k, n, 1)
    idx = np.array([9, 2, 15, 4, 11, 0], dtype=np.int32)
    y = _run_list(dev, x, w_nk, idx, prefix="unsorted", sort=False)
    assert_close(y, orc.gemm_ref64(x, w_nk, idx), "unsorted")
    xt = to_dev(x, dev).view(bt, 1, k)
    out = torch.empty(bt, 1, n, dtype=F16, device=dev)
    bsa._prepacked_block_sparse_gemm_from_active_blocks(xt, to_dev(w_nk, dev), to_dev(idx, dev), out,
                                                        cache_prefix="limit", active_blocks_limit=3)
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx[:3]), "active_blocks_limit")


def test_duplicate_ids_accumulate_twice(dev):
    """A list entry is one accumulation (the naive kernel loops over list entries, KRN:708)."""
    bt, k, n = 4, 512, 64
    x, w_nk, _ = case(12, bt, k, n, 1)
    idx = np.array([3, 3, 6], dtype=np.int32)
    y = _run_list(dev, x, w_nk, idx, prefix="dup", sort=False)
    ref = orc.gemm_ref64(x, w_nk, [3]) * 2 + orc.gemm_ref64(x, w_nk, [6])
    assert_close(y, ref, "duplicates")


@pytest.mark.parametrize("bt,plan", [(64, (1, 48, 4, 2, 64, 7)), (64, (1, 48, 4, 4, 64, 7)),
                                     (37, (1, 32, 4, 2, 32, 7)), (5, (1, 32, 4, 4, 16, 7))])
def test_lds_activation_kind_skips_exactly(dev, bt, plan):
    """Kind 7 loads each block's activations into LDS slots that the next blocks reuse; a slot
    of a skipped entry (leading pad, out-of-range id) must hold zeros, not what the slot held
    before.  A launch on an all-Inf activation first leaves Inf in every slot of every compute
    unit's LDS; then Inf and NaN sit in blocks that are never active, the list repeats one id
    and names ids outside [0, nblk), and its length leaves pad slots in every wave.  Exactly the
    oracle's result on the listed blocks (duplicates twice), finite, and bit-identical on a
    repeat."""
    k, n = 64 * 40, 1100
    nblk = orc.nblk_of(k)
    x, w_nk, _ = case(41 + bt, bt, k, n, 1, "normal")
    # the poisoned blocks are ordinary ids that are simply not in the list
    x[:, 64 * 7:64 * 8] = np.inf
    x[: (bt + 1) // 2, 64 * 23 + 5] = np.nan
    rng = np.random.default_rng(bt)
    valid = np.setdiff1d(np.arange(nblk), [7, 23])
    keep = rng.choice(valid, size=13, replace=False)
    idx = np.concatenate([keep, [keep[2], -1, nblk, nblk + 40]]).astype(np.int32)
    rng.shuffle(idx)
    ref = orc.gemm_ref64(x, w_nk, keep) + orc.gemm_ref64(x, w_nk, [keep[2]])
    xt, it = to_dev(x, dev), to_dev(idx, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    p = bsa.Plan(*plan)
    outs = []
    for _ in range(2):
        junk = torch.empty((bt, n), dtype=F16, device=dev)
        bsa.gemm_packed(torch.full_like(xt, float("inf")), packed, n, to_dev(np.arange(nblk, dtype=np.int32), dev),
                        junk, plan=p, workspace_prefix="k7")
        out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        print(f"kind 7 plan={plan} bt={bt} poisoned inactive blocks", flush=True)
        used = bsa.gemm_packed(xt, packed, n, it, out, plan=p, workspace_prefix="k7")
        assert used.as_tuple() == p.as_tuple(), used
        torch.cuda.synchronize()
        outs.append(out)
    y = outs[0].float().cpu().numpy()
    assert np.isfinite(y).all()
    assert_close(y, ref, f"kind 7 {plan} bt={bt}")
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_dropin_prepared_call_rechecks_what_its_key_does_not_pin(dev):
    """A repeated drop-in call site takes a prepared launch (packed weight, plan and workspace of
    its first call).  Every change its key does not pin must still be honoured: new x and out
    tensors, a new list of the same length, an in-place weight update (re-pack), an x whose
    address is not 16-byte aligned (copied on the general path), a non-contiguous out (raises),
    and the unsorted / unsorted-as-given forms.  Each result is checked against the oracle."""
    from bsa_mi355x import runtime

    bt, k, n, na = 16, 11008, 4096, 86
    x, w_nk, idx = case(61, bt, k, n, na, "laplace")
    rng = np.random.default_rng(62)
    idx_u = rng.permutation(idx).astype(np.int32)
    wt = to_dev(w_nk, dev)
    it = to_dev(idx_u, dev)
    prefix = "prepared"

    def run(xn, ids, out=None, sort=True):
        xt = to_dev(xn, dev).view(bt, 1, k)
        out = torch.full((bt, 1, n), float("nan"), dtype=F16, device=dev) if out is None else out
        bsa._prepacked_block_sparse_gemm_from_active_blocks(xt, wt, ids, out, cache_prefix=prefix,
                                                            sort_active_blocks=sort)
        torch.cuda.synchronize()
        return out.view(bt, n).float().cpu().numpy()

    runtime.forget_prepared_calls()
    assert_close(run(x, it), orc.gemm_ref(x, w_nk, idx), "first call")
    assert any(key[0] == prefix for key in runtime._PREPARED), "the first call left no prepared launch"
    x2, _, _ = case(63, bt, k, n, 1, "laplace")
    assert_close(run(x2, it), orc.gemm_ref(x2, w_nk, idx), "prepared: new x and out")
    idx2 = np.sort(rng.choice(k // 64, na, replace=False)).astype(np.int32)
    assert_close(run(x2, to_dev(rng.permutation(idx2).astype(np.int32), dev)), orc.gemm_ref(x2, w_nk, idx2),
                 "prepared: new list")
    with torch.no_grad():
        wt.mul_(-0.5)
    w_half = (w_nk.astype(np.float32) * -0.5).astype(np.float16)
    assert_close(run(x2, it), orc.gemm_ref(x2, w_half, idx), "after an in-place weight update")
    # the same shape and strides at an address 8 bytes past 16-byte alignment
    base = torch.empty(bt * k + 4, dtype=F16, device=dev)
    xo = base[4:].view(bt, 1, k)
    xo.copy_(to_dev(x, dev).view(bt, 1, k))
    assert xo.data_ptr() % 16 == 8
    out = torch.full((bt, 1, n), float("nan"), dtype=F16, device=dev)
    bsa._prepacked_block_sparse_gemm_from_active_blocks(xo, wt, it, out, cache_prefix=prefix)
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref(x, w_half, idx), "unaligned x")
    big = torch.empty(bt, 2, n, dtype=F16, device=dev)
    run(x, it)
    with pytest.raises(ValueError):
        bsa._prepacked_block_sparse_gemm_from_active_blocks(to_dev(x, dev).view(bt, 1, k), wt, it, big[:, :1, :],
                                                            cache_prefix=prefix)
    # a list taken as given (no sort): the kernel sums in list order, the same blocks
    assert_close(run(x, it, sort=False), orc.gemm_ref(x, w_half, idx_u), "unsorted as given")
    assert_close(run(x, it, sort=False), orc.gemm_ref(x, w_half, idx_u), "unsorted as given, prepared")


def test_every_instantiated_tile(dev):
    """Every compiled (rows, cols, waves, depth) kernel, split-K 1 and 3 (kind 3: 1 only), fp16
    and bf16; bt=37 gives kind 3 (at most 8 rows per work-group) several row groups."""
    bt, k, n, na = 37, 4096, 1000, 29
    x, w_nk, idx = case(13, bt, k, n, na)
    ref = orc.gemm_ref64(x, w_nk, idx)
    xb = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    wb = torch.from_numpy(w_nk.astype(np.float32)).to(torch.bfloat16)
    ref_bf = orc.gemm_ref64(xb.float().numpy(), wb.float().numpy(), idx)
    tiles = bsa.kernel_tiles()
    assert len(tiles) >= 60
    xt = to_dev(x, dev)
    it = to_dev(idx, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    packed_b = bsa.pack_weight(wb.to(dev))
    for kind, rows, cols, waves, depth in tiles:
        for sk in ((1,) if kind in (3, 5, 6, 7) else (1, 3)):
            # explicit plan through gemm_packed, so rows_per_group is honoured even when < bt
            out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
            p = bsa.Plan(sk, cols, waves, depth, rows, kind)
            print(f"tile kind={kind} rows={rows} cols={cols} waves={waves} depth={depth} split_k={sk}", flush=True)
            bsa.gemm_packed(xt, packed, n, it, out, plan=p, workspace_prefix="tiles")
            torch.cuda.synchronize()
            assert_close(out.float().cpu().numpy(), ref, f"tile {kind},{rows},{cols},{waves},{depth} sk={sk}")
        # bf16 once per tile (split-K 2)
        out_b = torch.full((bt, n), float("nan"), dtype=torch.bfloat16, device=dev)
        bsa.gemm_packed(xb.to(dev), packed_b, n, it, out_b,
                        plan=bsa.Plan(1 if kind in (3, 5, 6, 7) else 2, cols, waves, depth, rows, kind),
                        workspace_prefix="tiles_bf")
        torch.cuda.synchronize()
        yb = out_b.float().cpu().numpy()
        # bf16 output keeps 8 significant bits: tolerance 5e-3 rel. Frobenius, 2e-2 max-abs
        rf = orc.rel_frobenius(yb, ref_bf)
        assert rf <= 5e-3 and np.max(np.abs(yb - ref_bf)) <= 2e-2 * np.max(np.abs(ref_bf)), \
            f"bf16 tile {kind},{rows},{cols},{waves},{depth}: rel_fro={rf:.3e}"


@pytest.mark.parametrize("bt,rows,n_keep", [(1, 1, 34), (3, 4, 172), (4, 4, 172), (8, 8, 40)])
def test_dot_product_kernel(dev, bt, rows, n_keep):
    """Kind 3 (fp32 dot products, activations staged in LDS): the down shape dense at 4 rows
    stages 88 KiB of activations (above 64 KiB of LDS)."""
    k, n = 11008, 4096
    x, w_nk, idx = case(31 + bt, bt, k, n, n_keep)
    xt, it = to_dev(x, dev), to_dev(idx, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
    pl = bsa.gemm_packed(xt, packed, n, it, out, plan=bsa.Plan(0, 0, 0, 0, 0, 3), workspace_prefix="dot")
    torch.cuda.synchronize()
    assert (pl.kind, pl.rows_per_group) == (3, rows)
    assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx), f"kind 3 bt={bt} na={n_keep}")


@pytest.mark.parametrize("split_k", [1, 2, 4, 7, 16, 29])
def test_split_k_factors(dev, split_k):
    bt, k, n, na = 16, 11008, 4096, 86
    x, w_nk, idx = case(1234, bt, k, n, na)
    y = _run_list(dev, x, w_nk, idx, plan=dict(num_split_k=split_k), prefix=f"sk{split_k}")
    assert_close(y, orc.gemm_ref(x, w_nk, idx), f"split_k={split_k}")


def test_bitmap_and_dense_paths(dev):
    bt, k, n, na = 16, 4096, 2048, 23
    x, w_nk, idx = case(14, bt, k, n, na)
    nb = orc.nblk_of(k)
    xt = to_dev(x, dev).view(bt, 1, k)
    wt = to_dev(w_nk, dev)
    it = to_dev(idx, dev)
    out = torch.empty(bt, 1, n, dtype=F16, device=dev)
    bm = bsa._build_active_k_bitmap(it, nb, dev)
    assert np.array_equal(bm.cpu().numpy(), orc.bitmap_from_list(idx, nb))
    bsa._prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload(xt, wt, it, out, total_k_blocks=nb,
                                                                        prebuilt_bitmap=bm)
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx), "bitmap")
    bsa._prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload_splitk(xt, wt, it, out, total_k_blocks=nb,
                                                                               prebuilt_bitmap=bm, num_split_k=4)
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx), "bitmap split-K")
    # a shorter bitmap than ceil(K/64): later blocks are inactive
    bsa._prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload(xt, wt, it, out, total_k_blocks=40,
                                                                        prebuilt_bitmap=bm[:40].contiguous())
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx[idx < 40]), "short bitmap")
    bsa.dense_gemm(xt, wt, out)
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.arange(nb)), "dense")


def test_device_count(dev):
    """List capacity 40, device-side count 17: only the first 17 entries count."""
    bt, k, n = 16, 4096, 512
    x, w_nk, _ = case(15, bt, k, n, 1)
    rng = np.random.default_rng(3)
    idx = rng.permutation(64)[:40].astype(np.int32)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    out = torch.empty(bt, n, dtype=F16, device=dev)
    cnt = torch.tensor([17], dtype=torch.int32, device=dev)
    bsa.gemm_packed(to_dev(x, dev), packed, n, to_dev(idx, dev), out, num_active=40, num_active_dev=cnt)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx[:17]), "device count")


@pytest.mark.parametrize("plan", [(1, 16, 4, 4, 16, 1), (3, 16, 2, 4, 16, 1), (2, 16, 4, 4, 16, 2),
                                  (1, 16, 4, 4, 16, 4), (1, 48, 4, 4, 16, 5), (1, 48, 4, 4, 16, 6),
                                  (1, 32, 4, 4, 16, 7), (1, 32, 4, 2, 32, 7)])
def test_device_count_every_kind(dev, plan):
    """The device-side count in every MFMA kernel kind: counts below, at and above the list's
    capacity (clamped to it) and negative (no block: zeros), each launch on the same plan and
    workspace, against the oracle on the entries that count."""
    bt, k, n, cap = 16, 4096, 1000, 40
    x, w_nk, _ = case(16, bt, k, n, 1, "normal")
    rng = np.random.default_rng(4)
    idx = rng.permutation(64)[:cap].astype(np.int32)
    xt, it = to_dev(x, dev), to_dev(idx, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    p = bsa.Plan(*plan)
    for d in (17, cap, 55, 0, -3, 1):
        out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        cnt = torch.tensor([d], dtype=torch.int32, device=dev)
        print(f"device count plan={plan} count={d}", flush=True)
        used = bsa.gemm_packed(xt, packed, n, it, out, plan=p, num_active=cap, num_active_dev=cnt,
                               workspace_prefix="devcnt")
        assert used.as_tuple() == p.as_tuple(), used
        torch.cuda.synchronize()
        keep = idx[:max(0, min(d, cap))]
        y = out.float().cpu().numpy()
        if keep.size == 0:
            assert np.count_nonzero(y) == 0, (plan, d)
        else:
            assert_close(y, orc.gemm_ref64(x, w_nk, keep), f"plan {plan} count {d}")


def test_pack_layout_bit_exact(dev):
    """Device packing == oracle tile_permute(pack_kmajor(W)) bit for bit (both layouts)."""
    for n, k in ((100, 1000), (4096, 256), (48, 64)):
        rng = np.random.default_rng(n + k)
        w_nk = rng.normal(0, 0.02, size=(n, k)).astype(np.float16)
        want = orc.tile_permute(orc.pack_kmajor(w_nk))
        got = bsa.pack_weight(to_dev(w_nk, dev)).cpu().numpy()
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), (n, k)
        got_kn = bsa.pack_weight(to_dev(np.ascontiguousarray(w_nk.T), dev), layout="kn").cpu().numpy()
        assert np.array_equal(got_kn.view(np.uint16), want.view(np.uint16)), (n, k, "kn")
        # the reference-named accessor: the cached tiled tensor, guarded against reference-layout
        # slicing, and its block_major() view equal to the reference packing bit for bit
        tp = bsa._get_prepacked_weight_block_major(to_dev(w_nk, dev), 64, cache_prefix="packacc")
        assert isinstance(tp, bsa.TiledPackedWeight) and tuple(tp.shape) == want.shape
        with pytest.raises(TypeError):
            tp[0]
        bm = tp.block_major(n).cpu().numpy()
        assert np.array_equal(bm.view(np.uint16), orc.pack_kmajor(w_nk).view(np.uint16)), (n, k, "block_major")


@pytest.mark.parametrize("plan", [(8, 16, 2, 4, 16, 1), (8, 16, 4, 4, 16, 2), (8, 16, 8, 4, 64, 4), (8, 32, 8, 4, 64, 4)])
def test_split_k_more_splits_than_blocks(dev, plan):
    """Split-K 8 over 3 (then 1, then 0) active blocks: most work-groups' slices are empty, so
    the last arriver's own split is often all zeros and it loads the others'.  One workspace
    for every call, so each call also checks that the previous one re-armed the counters."""
    bt, k, n = 40, 4096, 1000
    x, w_nk, idx = case(29, bt, k, n, 3)
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    pl = bsa.Plan(*plan)
    for sub in (idx, idx[1:2], idx[:0]):
        out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        print(f"split-K 8 plan={plan} na={len(sub)}", flush=True)
        bsa.gemm_packed(xt, packed, n, to_dev(np.ascontiguousarray(sub), dev), out, plan=pl, workspace_prefix="sk_sparse")
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), orc.gemm_ref(x, w_nk, sub), f"plan {plan} na={len(sub)}")


def test_deterministic_repeats(dev):
    bt, k, n, na = 16, 11008, 4096, 62
    x, w_nk, idx = case(16, bt, k, n, na)
    a = _run_list(dev, x, w_nk, idx, plan=dict(num_split_k=8), prefix="det")
    b = _run_list(dev, x, w_nk, idx, plan=dict(num_split_k=8), prefix="det")
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


LLAMA = {"qkvo": (4096, 4096), "gate_up": (4096, 11008), "down": (11008, 4096)}


@pytest.mark.parametrize("bt,s", [(2, 0.803), (16, 0.638), (64, 0.520)])
@pytest.mark.parametrize("shape", ["qkvo", "gate_up", "down"])
def test_llama_shapes(dev, shape, bt, s):
    """every Llama-2-7B projection shape at its batch/sparsity pair."""
    k, n = LLAMA[shape]
    nb = orc.nblk_of(k)
    na = orc.n_active_for_sparsity(s, nb)
    x, w_nk, idx = case(1234, bt, k, n, na, "laplace" if shape == "down" else "normal")
    assert_close(_run_list(dev, x, w_nk, idx, prefix=f"llama_{shape}"), orc.gemm_ref(x, w_nk, idx),
                 f"{shape} B={bt} s={s}")


@pytest.mark.parametrize("s", [0.0, 0.25, 0.5, 0.638, 0.8])
def test_down_proj_sparsity_sweep(dev, s):
    """down_proj B=16 over the sparsity sweep (0 runs the dense path)."""
    k, n, bt = 11008, 4096, 16
    na = orc.n_active_for_sparsity(s, 172)
    x, w_nk, idx = case(1234, bt, k, n, na)
    if s == 0.0:
        xt = to_dev(x, dev).view(bt, 1, k)
        out = torch.empty(bt, 1, n, dtype=F16, device=dev)
        bsa.dense_gemm(xt, to_dev(w_nk, dev), out)
        torch.cuda.synchronize()
        y = out.view(bt, n).float().cpu().numpy()
    else:
        y = _run_list(dev, x, w_nk, idx, prefix="sweep")
    assert_close(y, orc.gemm_ref(x, w_nk, idx), f"down s={s}")


@pytest.mark.parametrize("plan", [
    (3, 16, 1, 4, 16, 1), (3, 16, 2, 4, 16, 1), (3, 16, 4, 4, 16, 1), (3, 16, 8, 4, 16, 1),  # kind 1, 64-512 threads
    (3, 32, 2, 4, 32, 1),
    (3, 16, 4, 4, 16, 2), (3, 16, 2, 4, 32, 2), (3, 16, 8, 4, 64, 2),  # kind 2
    (3, 16, 8, 4, 64, 4), (3, 16, 4, 4, 32, 4),                        # kind 4
    (1, 16, 4, 4, 2, 3), (1, 16, 8, 4, 2, 3),                          # kind 3
])
def test_block_sources_every_work_group_size(dev, plan):
    """Bitmap (compacted by a work-group scan whose width is the kernel's thread count), list
    with a device-side count, and dense, for every kernel kind and work-group size, split-K 3
    where the kind has it; bt=37 spans several row groups."""
    bt, k, n = 37, 11008, 1000
    nb = orc.nblk_of(k)
    x, w_nk, _ = case(17, bt, k, n, 1)
    rng = np.random.default_rng(plan[2] * 100 + plan[5])
    bm = (rng.random(nb) < 0.6).astype(np.uint8)
    lst = rng.permutation(nb)[:120].astype(np.int32)
    p = bsa.Plan(*plan)
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    out = torch.empty(bt, n, dtype=F16, device=dev)
    bsa.gemm_packed(xt, packed, n, None, out, bitmap=to_dev(bm, dev), plan=p, workspace_prefix="srcs")
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.flatnonzero(bm)), f"bitmap {plan}")
    cnt = torch.tensor([77], dtype=torch.int32, device=dev)
    bsa.gemm_packed(xt, packed, n, to_dev(lst, dev), out, num_active=120, num_active_dev=cnt, plan=p,
                    workspace_prefix="srcs")
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, lst[:77]), f"device count {plan}")
    bsa.gemm_packed(xt, packed, n, None, out, plan=p, workspace_prefix="srcs")
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.arange(nb)), f"dense {plan}")


def test_maximum_block_count(dev):
    """K = 64 * 2048, the most K-blocks the kernels take (BSG_MAX_NBLK): every block as a
    permuted list, as a bitmap and dense; the exact-L1 selector ranks all 2048 blocks."""
    bt, k, n = 3, 64 * 2048, 48
    nb = orc.nblk_of(k)
    assert nb == 2048
    x, w_nk, _ = case(18, bt, k, n, 1)
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    out = torch.empty(bt, n, dtype=F16, device=dev)
    want = orc.gemm_ref64(x, w_nk, np.arange(nb))
    perm = np.random.default_rng(5).permutation(nb).astype(np.int32)
    bsa.gemm_packed(xt, packed, n, to_dev(perm, dev), out, workspace_prefix="maxblk")
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), want, "2048-block list")
    bsa.gemm_packed(xt, packed, n, None, out, bitmap=torch.ones(nb, dtype=torch.uint8, device=dev),
                    workspace_prefix="maxblk")
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), want, "2048-block bitmap")
    bsa.gemm_packed(xt, packed, n, None, out, workspace_prefix="maxblk")
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), want, "2048-block dense")
    idx, cnt = bsa.select_topk_l1(xt, 1000, workspace_prefix="maxblk_sel")
    torch.cuda.synchronize()
    assert int(cnt.item()) == 1000
    assert np.array_equal(idx.cpu().numpy()[:1000], orc.select_topk_l1(x, 1000))


SORT_LISTS = {
    "random": np.random.default_rng(21).permutation(64)[:29],
    "descending": np.arange(63, 5, -2),
    "ascending": np.arange(3, 64, 3),
    "duplicates": np.array([5, 3, 5, 60, 0, 3, 3]),
    "out_of_range": np.array([7, -3, 64, 2, 1000, 7, -2147483648, 2147483647]),
    "single": np.array([42]),
}


@pytest.mark.parametrize("plan", [(1, 16, 2, 4, 16, 1), (3, 16, 4, 4, 32, 2), (2, 16, 8, 4, 64, 4), (1, 16, 4, 4, 4, 3),
                                  (1, 48, 4, 4, 16, 5), (1, 16, 4, 4, 16, 6)])
def test_in_kernel_sort_matches_sort_then_gemm(dev, plan):
    """bsg_gemm_sorted (the list sorted in the GEMM's own staging) gives, bit for bit, what an
    ascending sort of the list followed by bsg_gemm gives (KRN:3193-3194 then KRN:684-733), for
    unsorted, descending, already ascending, duplicated and out-of-range lists, on every kernel
    kind; a device count sorts only the first entries it names."""
    bt, k, n = 8, 4096, 1000
    x, w_nk, _ = case(22, bt, k, n, 1)
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    p = bsa.Plan(*plan)
    for name, ids in SORT_LISTS.items():
        ids = ids.astype(np.int32)
        print(f"in-kernel sort plan={plan} list={name} na={ids.size}", flush=True)
        got = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        want = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        bsa.gemm_packed(xt, packed, n, to_dev(ids, dev), got, plan=p, workspace_prefix="isort", sort_list=True)
        bsa.gemm_packed(xt, packed, n, to_dev(np.sort(ids), dev), want, plan=p, workspace_prefix="isort_ref")
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{name}: in-kernel sort differs from sort + GEMM"
        valid = ids[(ids >= 0) & (ids < 64)]
        assert_close(got.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.sort(valid)), f"sorted {name}")
    ids = SORT_LISTS["random"].astype(np.int32)[:20]
    got = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
    bsa.gemm_packed(xt, packed, n, to_dev(ids, dev), got, num_active=20,
                    num_active_dev=to_dev(np.array([12], dtype=np.int32), dev), plan=p, workspace_prefix="isort",
                    sort_list=True)
    torch.cuda.synchronize()
    assert_close(got.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.sort(ids[:12])), "device count")


def test_in_kernel_sort_bf16(dev):
    """The in-kernel sort is dtype-blind: bf16 inputs give, bit for bit, the GEMM on the sorted list."""
    bt, k, n = 16, 4096, 512
    x, w_nk, _ = case(26, bt, k, n, 1)
    xb = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).to(dev)
    packed = bsa.pack_weight(torch.from_numpy(w_nk.astype(np.float32)).to(torch.bfloat16).to(dev))
    ids = SORT_LISTS["random"].astype(np.int32)
    for plan in ((1, 16, 2, 4, 16, 1), (1, 16, 4, 4, 16, 6)):
        got = torch.full((bt, n), float("nan"), dtype=torch.bfloat16, device=dev)
        want = torch.full((bt, n), float("nan"), dtype=torch.bfloat16, device=dev)
        bsa.gemm_packed(xb, packed, n, to_dev(ids, dev), got, plan=bsa.Plan(*plan), workspace_prefix="isort_bf",
                        sort_list=True)
        bsa.gemm_packed(xb, packed, n, to_dev(np.sort(ids), dev), want, plan=bsa.Plan(*plan),
                        workspace_prefix="isort_bf_ref")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"bf16 in-kernel sort, plan {plan}"


def test_in_kernel_sort_at_its_limit_and_past_it(dev):
    """1024 entries (MAX_NBLK // 2, the in-kernel sort's limit) sorted in the GEMM; the drop-in
    sorts a longer list with a sort launch first (same result)."""
    bt, k, n = 3, 64 * 2048, 48
    x, w_nk, _ = case(23, bt, k, n, 1)
    xt = to_dev(x, dev)
    wt = to_dev(w_nk, dev)
    packed = bsa.pack_weight(wt)
    perm = np.random.default_rng(6).permutation(2048).astype(np.int32)
    got = torch.empty(bt, n, dtype=F16, device=dev)
    want = torch.empty(bt, n, dtype=F16, device=dev)
    bsa.gemm_packed(xt, packed, n, to_dev(perm[:1024], dev), got, workspace_prefix="isort_max", sort_list=True)
    bsa.gemm_packed(xt, packed, n, to_dev(np.sort(perm[:1024]), dev), want, workspace_prefix="isort_max_ref")
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert_close(got.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.sort(perm[:1024])), "1024 sorted in-kernel")
    with pytest.raises(ValueError):
        bsa.gemm_packed(xt, packed, n, to_dev(perm[:1025], dev), got, workspace_prefix="isort_max", sort_list=True)
    out = torch.empty(bt, 1, n, dtype=F16, device=dev)
    bsa._prepacked_block_sparse_gemm_from_active_blocks(xt.view(bt, 1, k), wt, to_dev(perm[:1500], dev), out,
                                                        cache_prefix="isort_long")
    torch.cuda.synchronize()
    assert_close(out.view(bt, n).float().cpu().numpy(), orc.gemm_ref64(x, w_nk, np.sort(perm[:1500])),
                 "1500 sorted by a sort launch")


@pytest.mark.parametrize("k,plan", [
    (4096, (1, 16, 2, 4, 16, 1)), (4096, (3, 16, 4, 4, 32, 2)), (4096, (2, 16, 8, 4, 64, 4)),
    (4096, (1, 16, 4, 4, 4, 3)), (4096, (1, 48, 4, 4, 16, 5)), (4096, (1, 48, 2, 4, 64, 6)),
    (4096, (1, 48, 4, 2, 64, 7)), (4096, (1, 32, 8, 2, 32, 7)),
    # K not a multiple of 64: the last block holds 40 or 8 channels, the rest of it is NaN padding
    (1000, (1, 16, 2, 4, 16, 1)), (1000, (1, 48, 4, 4, 16, 5)), (1000, (1, 48, 2, 4, 64, 6)),
    (1000, (1, 48, 4, 2, 64, 7)), (1032, (1, 32, 4, 4, 16, 7)), (1032, (2, 16, 4, 4, 32, 2)),
])
def test_strided_rows_and_side_stream(dev, k, plan):
    """X and Y as row-strided views (ldx > K, ldy > N), launched on a side stream: the padding
    columns of X hold NaN (any read past K would poison Y) and those of Y keep a sentinel."""
    bt, n = 40, 1000
    na = min(25, orc.nblk_of(k))
    x, w_nk, idx = case(19, bt, k, n, na)
    if k % 64 and orc.nblk_of(k) - 1 not in idx:
        idx = np.sort(np.append(idx[1:], orc.nblk_of(k) - 1)).astype(np.int32)  # the partial block counts
    x_wide = torch.full((bt, k + 64), float("nan"), dtype=F16, device=dev)
    x_wide[:, :k] = to_dev(x, dev)
    y_wide = torch.full((bt, n + 24), 7.0, dtype=F16, device=dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    it = to_dev(idx, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        bsa.gemm_packed(x_wide[:, :k], packed, n, it, y_wide[:, :n], plan=bsa.Plan(*plan), workspace_prefix="strided")
    s.synchronize()
    y = y_wide.float().cpu().numpy()
    assert np.all(y[:, n:] == 7.0), "columns past N were written"
    assert_close(y[:, :n], orc.gemm_ref64(x, w_nk, idx), f"strided K={k} {plan}")


@pytest.mark.parametrize("bt,plan", [
    (5, (1, 16, 4, 4, 16, 1)),    # kind 1: 4 waves, each its own slice
    (5, (3, 16, 2, 8, 16, 1)),    # kind 1 under split-K 3, depth 8
    (20, (2, 16, 4, 8, 32, 2)),   # kind 2: waves share the slice (per-block barrier)
    (40, (1, 16, 8, 4, 64, 4)),   # kind 4
    (3, (1, 16, 4, 4, 4, 3)),     # kind 3
    (9, (1, 48, 4, 4, 16, 5)),    # kind 5
    (50, (1, 48, 2, 4, 64, 6)),   # kind 6
    (50, (1, 48, 4, 2, 64, 7)),   # kind 7 (activations through LDS)
    (20, (1, 32, 4, 4, 32, 7)),
])
def test_pipeline_every_slice_length(dev, bt, plan):
    """Each wave's slice is rounded up to the prefetch depth with leading out-of-range slots and
    the last pass only drains: every active count from 0 to past 2 x waves x depth, so every
    slice length mod depth (and slices shorter than the depth) occurs in every kernel kind."""
    k, n = 64 * 48, 112
    nblk = orc.nblk_of(k)
    x, w_nk, _ = case(31 + bt, bt, k, n, 1, "normal")
    xt = to_dev(x, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    p = bsa.Plan(*plan)
    splitters = p.split_k * (p.waves_per_group if p.kind in (1, 3) else 1) * \
        (p.waves_per_group // 2 if p.kind == 5 else (p.waves_per_group if p.kind in (6, 7) else 1))
    top = min(nblk, 2 * splitters * p.depth + p.depth + 1)
    rng = np.random.default_rng(bt)
    for na in range(0, top + 1):
        idx = np.sort(rng.choice(nblk, size=na, replace=False)).astype(np.int32)
        out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        print(f"pipeline plan={plan} bt={bt} na={na}", flush=True)
        used = bsa.gemm_packed(xt, packed, n, to_dev(idx, dev) if na else torch.empty(0, dtype=torch.int32, device=dev),
                               out, plan=p, workspace_prefix="pipe")
        assert used.as_tuple() == p.as_tuple(), used
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), orc.gemm_ref64(x, w_nk, idx), f"plan {plan} na={na}")


@pytest.mark.parametrize("bt,k,n,na", [(64, 4096, 11008, 31), (37, 4096, 11008, 23), (16, 4096, 11008, 23),
                                       (2, 4096, 11008, 13), (64, 11008, 4096, 83), (33, 4096, 12288, 31),
                                       (16, 4096, 22016, 31), (5, 1000, 1000, 7)])
def test_variable_width_column_groups(dev, bt, k, n, na):
    """Kinds 5 and 6 deal N/16 subtiles to the work-groups as evenly as possible (2 or 3 each at
    N=11008 on 256 compute units, 1-6 elsewhere): every subtile written exactly once, list, dense
    and bitmap modes, against the oracle; repeated launches are bit-identical."""
    x, w_nk, idx = case(77 + bt, bt, k, n, na, "normal")
    xt, it = to_dev(x, dev), to_dev(idx, dev)
    packed = bsa.pack_weight(to_dev(w_nk, dev))
    ref = orc.gemm_ref64(x, w_nk, idx)
    rows = 16 if bt <= 16 else (32 if bt <= 32 else 64)
    k6 = {16: ((6, 48, 2, 4), (6, 48, 4, 4), (7, 32, 4, 4)), 32: ((6, 48, 2, 4), (6, 48, 4, 2), (7, 48, 4, 2)),
          64: ((6, 48, 2, 2), (6, 48, 4, 2), (7, 48, 4, 2), (7, 48, 4, 4))}
    for kind, cols, waves, depth in ((5, 48, 4, 4), (5, 32, 2, 4), (5, 96, 2, 4), (5, 16, 4, 4)) + k6[rows]:
        p = bsa.Plan(1, cols, waves, depth, rows, kind)
        out = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        print(f"kind {kind} bt={bt} K={k} N={n} plan={p.as_tuple()}", flush=True)
        used = bsa.gemm_packed(xt, packed, n, it, out, plan=p, workspace_prefix="vt")
        assert used.as_tuple() == p.as_tuple(), used
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), ref, f"kind {kind} {p.as_tuple()} bt={bt} N={n}")
        again = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        bsa.gemm_packed(xt, packed, n, it, again, plan=p, workspace_prefix="vt")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    # dense and bitmap modes (the list built on the device) in each kind
    bm = torch.zeros(orc.nblk_of(k), dtype=torch.uint8, device=dev)
    bm[it.long()] = 1
    ref_dense = orc.gemm_ref64(x, w_nk, np.arange(orc.nblk_of(k)))
    for kind, cols, waves, depth in ((5, 48, 4, 4), (6, 48, 2, 4), (7, 32, 4, 4 if rows == 16 else 2)):
        p = bsa.Plan(1, cols, waves, depth, rows, kind)
        dense = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        bsa.gemm_packed(xt, packed, n, None, dense, plan=p, workspace_prefix="vt")
        bout = torch.full((bt, n), float("nan"), dtype=F16, device=dev)
        bsa.gemm_packed(xt, packed, n, None, bout, bitmap=bm, plan=p, workspace_prefix="vt")
        torch.cuda.synchronize()
        assert_close(dense.float().cpu().numpy(), ref_dense, f"kind {kind} dense")
        assert_close(bout.float().cpu().numpy(), ref, f"kind {kind} bitmap")
