"""Pins the CPU oracle (no GPU): golden fixtures written by independent pure-Python loops,
closed forms, special cases and brute force, chosen so that a dropped term, a wrong index or a
transposed operand fails at least one of them."""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from oracle import bsg_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "gemm_*.npz"))))
def test_gemm_matches_golden_loops(path):
    d = np.load(path)
    y = orc.gemm_ref64(d["x"], d["w_nk"], d["idx"])
    np.testing.assert_allclose(y, d["y"], rtol=1e-12, atol=1e-12)
    y32 = orc.gemm_ref(d["x"], d["w_nk"], d["idx"])
    assert orc.within_tolerance(y32, d["y"]) or not np.any(d["y"])


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "select_*.npz"))))
def test_select_matches_golden_loops(path):
    d = np.load(path)
    assert np.array_equal(orc.select_topk_l1(d["x"], int(d["k"])), d["sel"])
    # exact integer scores equal the fp64 sums (fp16 |x| * 2^24 are exact integers)
    np.testing.assert_array_equal(orc.l1_scores(d["x"]).astype(np.float64), d["scores"] * 2.0 ** 24)


def test_golden_count():
    assert len(glob.glob(os.path.join(GOLDEN, "*.npz"))) >= 7


def test_pack_kmajor_closed_form():
    rng = np.random.default_rng(0)
    for n, k in ((5, 64), (7, 100), (16, 129)):
        w = rng.normal(size=(n, k)).astype(np.float16)
        wp = orc.pack_kmajor(w)
        nb = orc.nblk_of(k)
        assert wp.shape == (nb, 64, n)
        for j in range(nb):
            for c in range(64):
                kk = 64 * j + c
                want = w[:, kk] if kk < k else np.zeros(n, np.float16)
                assert np.array_equal(wp[j, c], want)


def test_tile_permute_index_formula_and_inverse():
    rng = np.random.default_rng(1)
    n, k = 40, 130
    w = rng.normal(size=(n, k)).astype(np.float16)
    ref = orc.pack_kmajor(w)
    t = orc.tile_permute(ref)
    npad = 48
    assert t.shape == (orc.nblk_of(k), npad // 16, 1024)
    flat = t.reshape(-1)
    for j in range(ref.shape[0]):
        for kk in range(64):
            for nn in range(npad):
                h, g, e = kk // 32, (kk % 32) // 8, kk % 8
                tt, c = nn // 16, nn % 16
                off = j * 64 * npad + tt * 1024 + h * 512 + g * 128 + c * 8 + e
                want = ref[j, kk, nn] if nn < n else 0
                assert flat[off] == want
    assert np.array_equal(orc.tile_unpermute(t, n), ref)


def test_gemm_dense_special_case():
    rng = np.random.default_rng(2)
    x = rng.normal(size=(3, 200)).astype(np.float16)
    w = rng.normal(size=(9, 200)).astype(np.float16)
    y = orc.gemm_ref64(x, w, np.arange(orc.nblk_of(200)))
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-12, atol=1e-12)


def test_gemm_single_block_and_empty():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(4, 256)).astype(np.float16)
    w = rng.normal(size=(6, 256)).astype(np.float16)
    y = orc.gemm_ref64(x, w, [2])
    np.testing.assert_allclose(y, x[:, 128:192].astype(np.float64) @ w[:, 128:192].astype(np.float64).T)
    assert not np.any(orc.gemm_ref64(x, w, []))
    assert not np.any(orc.gemm_ref(x, w, [4, 7, -1]))  # nblk = 4: all out of range


def test_gemm_permutation_invariance_and_not_transposed():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(5, 512)).astype(np.float16)
    w = rng.normal(size=(11, 512)).astype(np.float16)
    a = orc.gemm_ref64(x, w, [1, 4, 6])
    b = orc.gemm_ref64(x, w, [6, 1, 4])
    np.testing.assert_allclose(a, b, rtol=1e-12)
    assert a.shape == (5, 11)
    # one-hot activation picks a weight column: catches a transposed operand
    xo = np.zeros((1, 512), np.float16)
    xo[0, 64 * 4 + 3] = 1
    np.testing.assert_array_equal(orc.gemm_ref64(xo, w, [4])[0], w[:, 64 * 4 + 3].astype(np.float64))


def test_gemm_ref_torch_matches_numpy():
    x, w_kn, idx = orc.make_inputs(1234, 16, 1024, 256, "laplace", na=7)
    yt = orc.gemm_ref_torch(torch.from_numpy(x), torch.from_numpy(w_kn), torch.from_numpy(idx.astype(np.int64)))
    y = orc.gemm_ref64(x, np.ascontiguousarray(w_kn.T), idx)
    assert orc.within_tolerance(yt.numpy(), y)


def test_bitmap_round_trip():
    idx = np.array([5, 1, 9], np.int32)
    bm = orc.bitmap_from_list(idx, 12)
    assert bm.dtype == np.uint8 and bm.sum() == 3
    assert np.array_equal(orc.list_from_bitmap(bm), [1, 5, 9])


def test_f16_units_exact():
    vals = np.array([0.0, -0.0, 2 ** -24, 2 ** -14, 1.0, -1.5, 65504.0, 3.140625], dtype=np.float16)
    u = orc.f16_units(vals)
    np.testing.assert_array_equal(u.astype(np.float64), np.abs(vals.astype(np.float64)) * 2.0 ** 24)
    inf_nan = orc.f16_units(np.array([np.inf, np.nan], dtype=np.float16))
    assert inf_nan[0] > orc.f16_units(np.array([65504.0], np.float16))[0] and inf_nan[1] > inf_nan[0]


def test_l1_scores_brute_force():
    rng = np.random.default_rng(6)
    x = rng.laplace(0, 0.05, size=(3, 200)).astype(np.float16)
    s = orc.l1_scores(x)
    for j in range(4):
        want = sum(int(v) for v in orc.f16_units(x[:, 64 * j:min(64 * j + 64, 200)]).reshape(-1))
        assert int(s[j]) == want


def test_select_tie_rule_and_topk_agreement():
    x = np.zeros((2, 64 * 6), np.float16)
    x[:, 64 * 2:64 * 3] = 1.0
    x[:, 64 * 4:64 * 5] = 1.0
    x[:, 64 * 5:64 * 6] = 2.0
    assert np.array_equal(orc.select_topk_l1(x, 2), [2, 5])   # 5 strongest, then 2 beats 4 on id
    assert np.array_equal(orc.select_topk_l1(x, 4), [0, 2, 4, 5])
    assert np.array_equal(orc.select_topk_l1(np.zeros((1, 640), np.float16), 3), [0, 1, 2])
    # distinct scores: agrees with torch.topk on CPU
    rng = np.random.default_rng(7)
    x = rng.normal(size=(16, 4096)).astype(np.float16)
    s = torch.from_numpy(orc.l1_scores(x).astype(np.float64))
    assert len(set(s.tolist())) == s.numel()
    want = torch.topk(s, 23).indices.sort()[0].numpy()
    assert np.array_equal(orc.select_topk_l1(x, 23), want)


def test_n_keep_and_baseline_pairs():
    assert orc.n_keep(0.48, 64) == 31                # config 4: k=31 at ~0.52 sparsity
    assert orc.n_active_for_sparsity(0.5, 172) == 86  # config 1
    assert [orc.n_active_for_sparsity(s, 172) for s in (0, 0.25, 0.5, 0.638, 0.8)] == [172, 129, 86, 62, 34]
    assert [orc.n_active_for_sparsity(s, 64) for s in (0.803, 0.638, 0.520)] == [13, 23, 31]
    assert orc.n_keep(0.0, 64) == 1 and orc.n_keep(2.0, 64) == 64


def test_l2_mean_selector_reference_semantics():
    rng = np.random.default_rng(8)
    x = rng.normal(size=(4, 1000)).astype(np.float16)  # floor(1000/64) = 15 blocks
    got = orc.select_l2_mean_ref(x, 0.5)
    xb = torch.from_numpy(x[:, :960].astype(np.float32)).reshape(-1, 15, 64)
    want = torch.topk(xb.norm(dim=2).mean(dim=0), k=8).indices.sort()[0].numpy()
    assert np.array_equal(got, want)


def test_make_inputs_seeded():
    a = orc.make_inputs(1234, 2, 128, 32, "normal", na=1)
    b = orc.make_inputs(1234, 2, 128, 32, "normal", na=1)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    assert a[1].shape == (128, 32) and a[0].dtype == np.float16 and a[2].dtype == np.int32


@pytest.mark.parametrize("score,use_prior,use_scale", [("l2_mean", False, False), ("energy", False, False),
                                                       ("energy", False, True), ("l2_mean", True, False),
                                                       ("energy", True, True)])
@pytest.mark.parametrize("bt,kdim,k", [(1, 1024, 3), (4, 4096, 13), (16, 4096, 23), (64, 11008, 83), (7, 1000, 5)])
def test_scored_selector_matches_reference_formula(score, use_prior, use_scale, bt, kdim, k):
    """float64 restatement == the reference formula in torch float32 (topk / argsort) on inputs
    without near-ties; the partial block of K=1000 is never scored (floor(K/64) blocks)."""
    rng = np.random.default_rng(bt * 31 + k)
    x = rng.laplace(0, 0.05, size=(bt, kdim)).astype(np.float16)
    nb = kdim // 64
    prior = rng.uniform(0, 1, size=nb).astype(np.float32) if use_prior else None
    scale = rng.uniform(0.5, 2, size=kdim).astype(np.float32) if use_scale else None
    ids, keep, ratio = orc.select_scored_ref(x, k, score, prior=prior, alpha=0.7, eps=0.1, scale=scale)
    ids32, keep32, ratio32 = orc.select_scored_torch32(x, k, score, prior=prior, alpha=0.7, eps=0.1, scale=scale)
    assert keep == keep32 == min(k, nb) and np.array_equal(ids, ids32)
    assert abs(ratio - ratio32) <= 1e-5 * max(ratio, 1e-12)
    assert ids.max() < nb


def test_energy_budget_closed_form():
    """Block energies 32,16,8,4,4 per row (that many entries equal to 1, exact); k=1 keeps
    32/64 = 0.5 < 0.8, the cumulative energies 32,48,56,60,64 first reach 0.8*64 = 51.2 at
    rank 2, so blocks {0,1,2} stay, ratio 56/64."""
    x = np.zeros((3, 5 * 64), dtype=np.float16)
    for j, m in enumerate((32, 16, 8, 4, 4)):
        x[:, 64 * j:64 * j + m] = 1.0
    ids, keep, ratio = orc.select_scored_ref(x, 1, "energy", energy_keep=0.8)
    assert keep == 3 and np.array_equal(ids, [0, 1, 2]) and ratio == 56 / 64
    ids, keep, ratio = orc.select_scored_ref(x, 1, "energy", energy_keep=0.5)  # already met at k
    assert keep == 1 and np.array_equal(ids, [0]) and ratio == 0.5
    ids, keep, _ = orc.select_scored_ref(x, 2, "energy", energy_keep=1.0)  # everything
    assert keep == 5
    ids32, keep32, _ = orc.select_scored_torch32(x, 1, "energy", energy_keep=0.8)
    assert keep32 == 3 and np.array_equal(ids32, [0, 1, 2])


def test_scored_selector_ties_and_prior():
    """Equal scores go to the lower id; a prior reorders blocks by score * (prior + eps)^alpha."""
    x = np.ones((2, 4 * 64), dtype=np.float16)
    ids, _, _ = orc.select_scored_ref(x, 2, "l2_mean")
    assert np.array_equal(ids, [0, 1])
    ids, _, _ = orc.select_scored_ref(x, 2, "l2_mean", prior=np.array([0, 0, 1, 2], np.float32), alpha=1.0, eps=0.1)
    assert np.array_equal(ids, [2, 3])
    ids, _, _ = orc.select_scored_ref(x, 1, "energy", prior=np.array([-5, 0, 0, 0], np.float32), alpha=2.0, eps=0.1)
    assert np.array_equal(ids, [1])  # prior clamped to 1e-6 for block 0; ties among 1..3 -> 1


def test_prior_of_the_wrong_length_is_ignored():
    """RRD:110-112 applies block_prior only when it holds exactly total_k entries: a shorter or
    longer prior leaves the scores as without one, in both restatements."""
    rng = np.random.default_rng(8)
    x = rng.laplace(0, 0.05, size=(8, 4 * 64)).astype(np.float16)
    base = orc.select_scored_ref(x, 2, "l2_mean")
    base32 = orc.select_scored_torch32(x, 2, "l2_mean")
    for prior in (np.array([0, 0, 9], np.float32), np.array([0, 0, 9, 9, 9], np.float32)):
        got = orc.select_scored_ref(x, 2, "l2_mean", prior=prior)
        got32 = orc.select_scored_torch32(x, 2, "l2_mean", prior=prior)
        assert np.array_equal(got[0], base[0]) and np.array_equal(got32[0], base32[0])
    ids, _, _ = orc.select_scored_ref(x, 2, "l2_mean", prior=np.array([0, 0, 9, 9], np.float32))
    assert np.array_equal(ids, [2, 3])


def test_scored_ref_ranks_nan_first_and_negative_scores_last_like_torch():
    """A block whose score is NaN ranks above every number, as torch.topk ranks NaN (the
    reference's own call, RRD:113), and negative scores (a negative channel scale) rank below
    zero and positive ones: the float64 restatement agrees with the torch float32 one."""
    rng = np.random.default_rng(31)
    x = rng.normal(0, 1, size=(4, 8 * 64)).astype(np.float16)
    x[2, 64 * 5 + 7] = np.nan
    for score in ("l2_mean", "energy"):
        ids, keep, _ = orc.select_scored_ref(x, 3, score)
        ids32, keep32, _ = orc.select_scored_torch32(x, 3, score)
        assert 5 in ids and keep == keep32 == 3 and np.array_equal(ids, ids32), (score, ids, ids32)
    xf = rng.normal(0, 1, size=(4, 8 * 64)).astype(np.float16)
    scale = np.where(np.arange(8 * 64) // 64 % 2 == 0, 1.0, -1.0).astype(np.float32)  # odd blocks score < 0
    for k in (3, 5):
        ids, _, _ = orc.select_scored_ref(xf, k, "energy", scale=scale)
        ids32, _, _ = orc.select_scored_torch32(xf, k, "energy", scale=scale)
        assert np.array_equal(ids, ids32)
    assert np.array_equal(orc.select_scored_ref(xf, 4, "energy", scale=scale)[0], [0, 2, 4, 6])


def test_make_inputs_several_masks_equal_single_draws():
    """A list of counts gives, for each, the mask make_inputs draws for that count alone."""
    x, w, masks = orc.make_inputs(77, 3, 640, 48, "laplace", na=[2, 5, 10])
    for m, idx in zip((2, 5, 10), masks):
        x1, w1, i1 = orc.make_inputs(77, 3, 640, 48, "laplace", na=m)
        assert np.array_equal(x, x1) and np.array_equal(w, w1) and np.array_equal(idx, i1)


def test_replay_case_bookkeeping():
    """The per-step replay's cases follow BPS:84-87 and 124-135: density 1 - S clamped to
    [0, 1], floor(density * nblk) blocks (at least one), one distinct case per (shape, density)."""
    from bsa_mi355x import replay

    assert replay.density_tenths(7) == 3 and replay.density_tenths(0) == 10 and replay.density_tenths(12) == 0
    for nblk in (64, 172):
        for s_tenths in range(11):  # the reference's float path: floor((1.0 - S) * nblk), S as stored
            want = max(1, min(nblk, int(np.floor((1.0 - s_tenths / 10.0) * nblk))))
            assert replay.active_count(replay.density_tenths(s_tenths), nblk) == want, (nblk, s_tenths)
    assert replay.active_count(3, 64) == 19 and replay.active_count(5, 172) == 86 and replay.active_count(0, 64) == 1
    m = np.zeros((7, 32), np.uint8)
    m[6, :] = 8
    m[0, 0] = 9
    assert replay.unique_cases([m]) == [("down", 2), ("gate_up", 10), ("qkvo", 1), ("qkvo", 10)]
    d, s = replay.step_sums(m, {"qkvo": 1.0, "gate_up": 2.0, "down": 3.0},
                            {("down", 2): 0.5, ("gate_up", 10): 2.0, ("qkvo", 1): 0.1, ("qkvo", 10): 1.0})
    assert d == 4 * 32 * 1.0 + 2 * 32 * 2.0 + 32 * 3.0
    assert abs(s - (0.1 + 127 * 1.0 + 64 * 2.0 + 32 * 0.5)) < 1e-9
    fx = replay.load_maps(os.path.join(os.path.dirname(__file__), "golden", "perstep_smaps.npz"))
    cases = replay.cases_for_batches(fx, [2, 64], steps_per_batch=2)
    assert set(cases) == {2, 64} and all(len(v) > 0 for v in cases.values())


def test_perstep_fixture_matches_reference_summaries():
    """The S-map fixture (tests/golden/make_perstep_fixture.py, from the reference's result
    files) decodes to the mean sparsity the reference recorded for each group-step, and the
    reference's per-batch speedups are the means of its per-step ones."""
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "perstep_smaps.npz"), allow_pickle=False)
    maps = f["smap_tenths"].astype(np.float64) / 10.0
    assert maps.shape == (330, 7, 32) and maps.max() <= 0.9
    assert np.abs(maps.reshape(330, -1).mean(axis=1) - f["mean_sparsity"]).max() < 1e-12
    for b, s in zip(f["ref_batch"], f["ref_batch_speedup"]):
        sel = f["batch"] == b
        assert sel.sum() == 55 and abs(f["ref_step_speedup"][sel].mean() - s) < 1e-12
    assert [round(float(v), 3) for v in f["ref_batch_speedup"]] == [1.948, 1.945, 1.761, 1.602, 1.405, 1.203]


def test_gemm_2d_every_block_is_the_1d_gemm():
    rng = np.random.default_rng(21)
    bt, k, n = 3, 200, 150  # partial last K-block and output block
    x = rng.normal(size=(bt, k)).astype(np.float16)
    w = rng.normal(size=(n, k)).astype(np.float16)
    kb = [0, 2, 3]
    y = orc.gemm_ref(x, w, kb)
    allb = list(range(3))
    np.testing.assert_array_equal(orc.gemm_2d_ref(x, w, kb, allb, out_init=np.zeros((bt, n))), y)
    c = orc.gemm_2d_ref(x, w, kb, allb, compact=True)
    assert c.shape == (bt, 192)
    np.testing.assert_array_equal(c[:, :n], y)
    assert not np.any(c[:, n:])


def test_gemm_2d_brute_force_loops():
    """Pure-Python fp64 loops: a partial last output block, an unsorted list and an id past
    the last block (nothing in place, zeros when compact)."""
    rng = np.random.default_rng(22)
    bt, k, n = 2, 128, 130
    x = rng.normal(size=(bt, k)).astype(np.float16)
    w = rng.normal(size=(n, k)).astype(np.float16)
    kb, nb = [1], [2, 0, 7]
    init = np.full((bt, n), 5.0, dtype=np.float32)
    want = init.astype(np.float64).copy()
    wantc = np.zeros((bt, 64 * len(nb)))
    for r in range(bt):
        for i, b in enumerate(nb):
            for c in range(64):
                col = 64 * b + c
                if b > 2 or col >= n:
                    continue
                s = 0.0
                for j in kb:
                    for ch in range(64 * j, 64 * j + 64):
                        s += float(x[r, ch]) * float(w[col, ch])
                want[r, col] = s
                wantc[r, 64 * i + c] = s
    got = orc.gemm_2d_ref(x, w, kb, nb, out_init=init)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(orc.gemm_2d_ref(x, w, kb, nb, compact=True), wantc, rtol=1e-5, atol=1e-4)
    # the compact result scattered back is the in-place result
    comp = orc.gemm_2d_ref(x, w, kb, nb, compact=True)
    np.testing.assert_array_equal(orc.scatter_ref(comp, nb, init), got)


def test_nmask_blocks_brute_force():
    rng = np.random.default_rng(23)
    for n in (1, 64, 65, 1000, 4096):
        m = (rng.random(n) < 0.01).astype(np.uint8)
        want = [b for b in range((n + 63) // 64) if any(m[c] for c in range(64 * b, min(64 * b + 64, n)))]
        np.testing.assert_array_equal(orc.nmask_blocks_ref(m, n), np.array(want, dtype=np.int32))
    assert orc.nmask_blocks_ref(np.zeros(300, np.uint8), 300).size == 0
