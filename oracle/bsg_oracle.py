"""CPU oracle of the batch-shared 64-channel block-sparse GEMM path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the bsa_mi355x package, the HIP
library) imports or calls this module; only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg do, as the checker.

A restatement in numpy (and torch CPU for the BASELINE-defined CPU path) of the reference's
algorithm.  References are to /root/reference (read, never run):
  KRN = kernels/shared_mask_batched_triton_min_runtime.py
  RRD = scripts/bench_roundrobin_e2e_decode.py
  BPS = scripts/bench_perstep_actual_kernel_speedup.py

How each function is pinned (tests/test_oracle.py):
  pack_kmajor        closed form (transpose + zero pad + view) and element-wise identity
  tile_permute       inverse permutation round trip; every element of the MFMA fragment
                     order checked against the index formula written in include/bsgemm.h
  gemm_ref           pure-Python fp64 triple loop on tiny inputs (tests/golden/*.npz),
                     dense special case (all blocks = X·W), na=0 -> 0, na=1 -> one
                     [B,64]x[64,N] product, permutation invariance, out-of-range ids -> 0
  l1_units/scores    fp64 |x| sums x 2^24 (exact for fp16) and brute-force integer loops
  select_topk_l1     brute-force sort by (-score, id); constructed ties; torch.topk on
                     CPU when scores are distinct
  n_keep             RRD:102 rounding (Python round) on the BASELINE pairs (0.52 -> 31/64)
  gemm_2d_ref        every output block listed = gemm_ref (in place, and compact with the
                     tail padded); pure-Python fp64 loop on tiny inputs with a partial last
                     block and an out-of-range id; scatter_ref(compact) = in place
  nmask_blocks_ref   brute force over reshaped masks (any per 64 columns)
"""
from __future__ import annotations

import math

import numpy as np

BLOCK_K = 64  # KRN:17 INDEX_BLOCK_META_SIZE


def nblk_of(k: int) -> int:
    """ceil(K / 64) (KRN:3153)."""
    return (int(k) + BLOCK_K - 1) // BLOCK_K


def pack_kmajor(w_nk: np.ndarray) -> np.ndarray:
    """The reference packing: pad(W^T) to nblk*64 rows, view [nblk, 64, N] (KRN:3152-3161)."""
    n, k = w_nk.shape
    nblk = nblk_of(k)
    wt = np.zeros((nblk * BLOCK_K, n), dtype=w_nk.dtype)
    wt[:k, :] = w_nk.T
    return wt.reshape(nblk, BLOCK_K, n)


def tile_permute(wp_ref: np.ndarray) -> np.ndarray:
    """Reorder the reference's [nblk, 64, N] packing into this build's tiled K-major layout
    [nblk, Np/16, 1024]: element (j, k, n) -> [j, n//16, (k//32)*512 + ((k%32)//8)*128 +
    (n%16)*8 + k%8], N zero-padded to a multiple of 16 (layout of include/bsgemm.h)."""
    nblk, bk, n = wp_ref.shape
    assert bk == BLOCK_K
    npad = (n + 15) // 16 * 16
    w = np.zeros((nblk, BLOCK_K, npad), dtype=wp_ref.dtype)
    w[:, :, :n] = wp_ref
    # axes: j, h(2), g(4), e(8), t(npad/16), c(16)
    w6 = w.reshape(nblk, 2, 4, 8, npad // 16, 16)
    # target order: j, t, h, g, c, e
    return np.ascontiguousarray(w6.transpose(0, 4, 1, 2, 5, 3)).reshape(nblk, npad // 16, 1024)


def tile_unpermute(wt: np.ndarray, n: int) -> np.ndarray:
    """Inverse of tile_permute: [nblk, Np/16, 1024] -> [nblk, 64, n]."""
    nblk, ntile, _ = wt.shape
    w6 = wt.reshape(nblk, ntile, 2, 4, 16, 8)  # j, t, h, g, c, e
    w = w6.transpose(0, 2, 3, 5, 1, 4).reshape(nblk, BLOCK_K, ntile * 16)
    return np.ascontiguousarray(w[:, :, :n])


def active_columns(idx, k: int) -> np.ndarray:
    """Channel ids of the listed blocks, restricted to valid ones: 64*j + c with 0 <= j < nblk
    and 64*j + c < K.  The reference kernels mask rk < M (KRN:709-717), so a block id past
    the last block contributes nothing; negative ids are treated the same way here."""
    idx = np.asarray(idx, dtype=np.int64).reshape(-1)
    nb = nblk_of(k)
    idx = idx[(idx >= 0) & (idx < nb)]
    cols = (BLOCK_K * idx[:, None] + np.arange(BLOCK_K)[None, :]).reshape(-1)
    return cols[cols < k]


def gemm_ref(x: np.ndarray, w_nk: np.ndarray, idx) -> np.ndarray:
    """Y[bt, N] = X[:, cols(idx)] · W^T[cols(idx), :] in fp32 (KRN:684-733 semantics; the
    BASELINE CPU path: gather, convert to fp32, matmul).  Returns float32."""
    cols = active_columns(idx, x.shape[1])
    if cols.size == 0:
        return np.zeros((x.shape[0], w_nk.shape[0]), dtype=np.float32)
    xa = x[:, cols].astype(np.float32)
    wa = w_nk[:, cols].astype(np.float32)
    return xa @ wa.T


def gemm_ref64(x: np.ndarray, w_nk: np.ndarray, idx) -> np.ndarray:
    """Same as gemm_ref in float64 (the tolerance reference for fp16/bf16 outputs)."""
    cols = active_columns(idx, x.shape[1])
    if cols.size == 0:
        return np.zeros((x.shape[0], w_nk.shape[0]), dtype=np.float64)
    return x[:, cols].astype(np.float64) @ w_nk[:, cols].astype(np.float64).T


def gemm_ref_torch(x_t, w_kn_t, idx_t):
    """BASELINE-defined CPU reference path on torch CPU tensors: gather + fp32 matmul.
    x_t [bt, K] fp16, w_kn_t [K, N] fp16 (stored [K,N]), idx_t int64 block ids.  Returns fp32."""
    import torch

    cols = (BLOCK_K * idx_t[:, None] + torch.arange(BLOCK_K)[None, :]).reshape(-1)
    return x_t.index_select(1, cols).float() @ w_kn_t.index_select(0, cols).float()


BLOCK_N = 64  # KRN:19 INDEX_BLOCK_OUT_META_SIZE, the output-block width of the 2-D path


def gemm_2d_ref(x: np.ndarray, w_nk: np.ndarray, k_idx, n_idx, out_init=None, compact: bool = False) -> np.ndarray:
    """2-D block sparsity in fp32: Y = gemm_ref(x, w_nk, k_idx) restricted to the listed
    64-column output blocks (KRN:2289-2384 in place, KRN:2473-2557 compact).  In place: a copy
    of out_init [bt, N] with the listed blocks' columns (< N) replaced.  Compact: [bt, 64 *
    len(n_idx)], entry i at columns 64i.. (columns past N zero).  A block id outside
    [0, ceil(N/64)) writes nothing in place and zeros when compact (its weight columns are
    masked off, KRN:2371-2375, 2544-2548)."""
    y = gemm_ref(x, w_nk, k_idx)
    bt, n = y.shape
    nnb = (n + BLOCK_N - 1) // BLOCK_N
    n_idx = np.asarray(n_idx, dtype=np.int64).reshape(-1)
    if compact:
        out = np.zeros((bt, BLOCK_N * len(n_idx)), dtype=np.float32)
    else:
        out = np.array(out_init, dtype=np.float32, copy=True)
    for i, b in enumerate(n_idx):
        if b < 0 or b >= nnb:
            continue
        c0, c1 = BLOCK_N * b, min(BLOCK_N * (b + 1), n)
        if compact:
            out[:, BLOCK_N * i:BLOCK_N * i + (c1 - c0)] = y[:, c0:c1]
        else:
            out[:, c0:c1] = y[:, c0:c1]
    return out


def scatter_ref(compact: np.ndarray, n_idx, out_init: np.ndarray) -> np.ndarray:
    """out[:, 64 b_i + c] = compact[:, 64 i + c] for c < 64 and 64 b_i + c < N (KRN:3470-3495)."""
    out = np.array(out_init, copy=True)
    n = out.shape[1]
    for i, b in enumerate(np.asarray(n_idx, dtype=np.int64).reshape(-1)):
        if b < 0 or b >= (n + BLOCK_N - 1) // BLOCK_N:
            continue
        w = min(BLOCK_N, n - BLOCK_N * b)
        out[:, BLOCK_N * b:BLOCK_N * b + w] = compact[:, BLOCK_N * i:BLOCK_N * i + w]
    return out


def nmask_blocks_ref(mask: np.ndarray, n: int) -> np.ndarray:
    """Ascending ids of the 64-column blocks with any nonzero mask entry below N (the block
    counts of KRN:453-495 taken > 0)."""
    m = np.asarray(mask).reshape(-1)[:n] != 0
    return np.array([b for b in range((n + BLOCK_N - 1) // BLOCK_N) if m[BLOCK_N * b:BLOCK_N * (b + 1)].any()],
                    dtype=np.int32)


def bitmap_from_list(idx, total_k_blocks: int) -> np.ndarray:
    """u8 bitmap, 1 at each listed block (KRN:1056-1061)."""
    bm = np.zeros(int(total_k_blocks), dtype=np.uint8)
    idx = np.asarray(idx, dtype=np.int64)
    if idx.size:
        bm[idx] = 1
    return bm


def list_from_bitmap(bm) -> np.ndarray:
    """Ascending active ids of a bitmap: the order in which the bitmap kernel accumulates
    (KRN:845 loops block_id = 0..N_TOTAL_K_BLOCKS-1 and skips inactive blocks)."""
    return np.nonzero(np.asarray(bm) != 0)[0].astype(np.int32)


def f16_units(x: np.ndarray) -> np.ndarray:
    """|x| of fp16 values in integer units of 2^-24 (exact: every finite fp16 is a multiple
    of 2^-24).  Non-finite values map above every finite one (Inf = 1024 << 30, NaN larger),
    the same map the device selector uses."""
    b = np.asarray(x, dtype=np.float16).view(np.uint16).astype(np.uint64) & np.uint64(0x7FFF)
    e = b >> np.uint64(10)
    m = b & np.uint64(0x3FF)
    sh = np.where(e > 0, e - np.uint64(1), np.uint64(0))
    return np.where(e == 0, m, (np.uint64(1024) | m) << sh)


def l1_scores(x: np.ndarray) -> np.ndarray:
    """score_j = sum_b sum_{c in block j, 64j+c < K} |x[b, 64j+c]| in units of 2^-24 (uint64)."""
    bt, k = x.shape
    nb = nblk_of(k)
    u = f16_units(x)
    pad = np.zeros((bt, nb * BLOCK_K), dtype=np.uint64)
    pad[:, :k] = u
    return pad.reshape(bt, nb, BLOCK_K).sum(axis=(0, 2), dtype=np.uint64)


def select_topk_l1(x: np.ndarray, k: int) -> np.ndarray:
    """Top-k blocks by (score desc, block id asc), returned ascending as int32.
    BASELINE rule: np.lexsort((idx, -score)), take k, sort ascending."""
    s = l1_scores(x)
    nb = s.shape[0]
    kk = max(0, min(int(k), nb))
    # exact integer keys (uint64 does not survive negation in numpy): sort in Python ints
    order = sorted(range(nb), key=lambda j: (-int(s[j]), j))
    return np.sort(np.asarray(order[:kk], dtype=np.int64)).astype(np.int32)


def select_l2_mean_ref(x: np.ndarray, density: float) -> np.ndarray:
    """The reference's online selector (RRD:90-113): score_j = mean_b ||x_b[64j:64j+64]||_2 in
    fp32, n_keep = max(1, min(nblk, round(density*nblk))), top-k, ascending int32.  Blocks are
    floor(K/64) as in RRD:97-99.  Ties are broken by lower id here (torch.topk's tie order is
    unspecified)."""
    bt, kdim = x.shape
    total_k = kdim // BLOCK_K
    xb = x[:, : total_k * BLOCK_K].astype(np.float32).reshape(bt, total_k, BLOCK_K)
    score = np.sqrt((xb * xb).sum(axis=2)).mean(axis=0)
    nk = n_keep(density, total_k)
    order = sorted(range(total_k), key=lambda j: (-float(score[j]), j))
    return np.sort(np.asarray(order[:nk], dtype=np.int32))


def block_stats64(x: np.ndarray, scale=None):
    """Per whole block j < floor(K/64) (RRD:97-99), in float64: the batch mean of the per-row
    L2 norm (RRD:100), of the energy sum x^2 (RRD:131, 156), and of the channel-scaled energy
    sum x^2 * scale_c (RRD:103-105)."""
    bt, kdim = x.shape
    nb = kdim // BLOCK_K
    xb = np.asarray(x, dtype=np.float64)[:, : nb * BLOCK_K].reshape(bt, nb, BLOCK_K)
    sq = xb * xb
    l2 = np.sqrt(sq.sum(axis=2)).mean(axis=0)
    energy = sq.sum(axis=2).mean(axis=0)
    if scale is None:
        return l2, energy, energy
    sc = np.asarray(scale, dtype=np.float64)[: nb * BLOCK_K].reshape(1, nb, BLOCK_K)
    return l2, energy, (sq * sc).sum(axis=2).mean(axis=0)


def select_scored_ref(x: np.ndarray, k: int, score: str = "l2_mean", prior=None, alpha: float = 1.0,
                      eps: float = 0.1, scale=None, energy_keep: float = 0.0):
    """The reference's scoring rules (RRD:90-176) in float64, ranking by (score desc, id asc):
      score  = l2 (RRD:100) or energy [* scale] (RRD:103-105, 131), times
               max(prior + eps, 1e-6)^alpha when a prior of exactly nblk entries is given
               (RRD:106-112; a prior of any other length is ignored, as there);
      keep   = min(k, nblk), grown while energy_keep > 0 and the top-keep energy share is below
               it, to searchsorted(cum, energy_keep * total) + 1 clamped to [k, nblk] (RRD:165-176);
      ratio  = cumulative energy at keep / max(total, 1e-12) (RRD:141, 176).
    A NaN score ranks above every number (torch.topk's order for NaN) and -0 ties with +0.
    Returns (ids ascending int32, keep, ratio)."""
    l2, energy, es = block_stats64(x, scale)
    nb = len(energy)
    sc = (l2 if score == "l2_mean" else es).copy()
    if prior is not None and np.asarray(prior).size == nb:  # any other length is ignored (RRD:110-112)
        pr = np.asarray(prior, dtype=np.float64).reshape(-1) + float(eps)
        sc = sc * np.maximum(pr, 1e-6) ** float(alpha)
    order = sorted(range(nb), key=lambda j: (-math.inf if math.isnan(sc[j]) else -float(sc[j]), j))
    k0 = max(0, min(int(k), nb))
    cum = np.cumsum(energy[order])
    total = max(float(energy.sum()), 1e-12)
    keep = k0
    if energy_keep > 0 and k0 > 0 and cum[k0 - 1] / total < energy_keep:
        first = int(np.searchsorted(cum, energy_keep * total, side="left"))
        keep = max(k0, min(nb, first + 1))
    ratio = float(cum[keep - 1] / total) if keep > 0 else 0.0
    return np.sort(np.asarray(order[:keep], dtype=np.int32)), keep, ratio


def select_scored_torch32(x, k: int, score: str = "l2_mean", prior=None, alpha: float = 1.0, eps: float = 0.1,
                          scale=None, energy_keep: float = 0.0):
    """The same rules written the way the reference evaluates them: torch CPU float32,
    torch.topk / argsort / cumsum / searchsorted (RRD:97-113, 127-141, 151-176).  Pins
    select_scored_ref on inputs without near-ties (torch's tie order is unspecified)."""
    import torch

    x3 = torch.as_tensor(np.asarray(x)).reshape(x.shape[0], 1, x.shape[-1])
    total_k = x3.shape[-1] // BLOCK_K
    xb = x3[..., : total_k * BLOCK_K].float().reshape(-1, total_k, BLOCK_K)
    energy = xb.pow(2).sum(dim=2).mean(dim=0)
    if score == "l2_mean":
        sc = xb.norm(dim=2).mean(dim=0)
    elif scale is None:
        sc = energy
    else:
        sc = (xb.pow(2) * torch.as_tensor(np.asarray(scale, dtype=np.float32))[: total_k * BLOCK_K]
              .reshape(1, total_k, BLOCK_K)).sum(dim=2).mean(dim=0)
    if prior is not None and int(np.asarray(prior).size) == int(total_k):  # RRD:110-112
        sc = sc * torch.clamp(torch.as_tensor(np.asarray(prior, dtype=np.float32)) + float(eps), min=1e-6).pow(
            float(alpha))
    k0 = max(0, min(int(k), total_k))
    order = torch.argsort(sc, descending=True)
    cum = torch.cumsum(energy[order], dim=0)
    total = max(float(energy.sum().item()), 1e-12)
    keep = k0
    if energy_keep > 0 and k0 > 0 and float(cum[k0 - 1].item() / total) < float(energy_keep):
        first = int(torch.searchsorted(cum, torch.tensor(float(energy_keep) * total)).item())
        keep = max(k0, min(total_k, first + 1))
    ids = torch.topk(sc, k=keep).indices.sort()[0].to(torch.int32).numpy()
    ratio = float(cum[keep - 1].item() / total) if keep > 0 else 0.0
    return ids, keep, ratio


def n_keep(density: float, total_k: int) -> int:
    """max(1, min(total_k, round(density * total_k))) (RRD:102, Python's round)."""
    return max(1, min(int(total_k), int(round(float(density) * int(total_k)))))


def n_active_for_sparsity(sparsity: float, nblk: int) -> int:
    """na = round((1 - s) * nblk) (0.5 of 172 -> 86, 0.638 -> 62)."""
    return int(round((1.0 - float(sparsity)) * int(nblk)))


def make_inputs(seed: int, bt: int, k: int, n: int, x_dist: str = "laplace", na: int | None = None):
    """BASELINE synthetic inputs from numpy default_rng(seed) (PCG64), drawn in this order:
    W ~ N(0, 0.02) stored [K, N] (fp16), X ~ Laplace(0, 0.05) or N(0, 1) (fp16) of shape
    [bt, K], then the mask rng.choice(nblk, na, replace=False) sorted ascending (int32)."""
    rng = np.random.default_rng(seed)
    w_kn = rng.normal(0.0, 0.02, size=(k, n)).astype(np.float16)
    if x_dist == "laplace":
        x = rng.laplace(0.0, 0.05, size=(bt, k)).astype(np.float16)
    elif x_dist == "normal":
        x = rng.normal(0.0, 1.0, size=(bt, k)).astype(np.float16)
    else:
        raise ValueError(x_dist)
    nb = nblk_of(k)
    if na is None:
        na = nb
    if isinstance(na, (list, tuple)):
        # one mask per count, each drawn from the state right after X, so entry i equals the
        # mask of make_inputs(seed, bt, k, n, x_dist, na[i])
        state = rng.bit_generator.state
        out = []
        for m in na:
            rng.bit_generator.state = state
            out.append(np.sort(rng.choice(nb, size=int(m), replace=False)).astype(np.int32))
        return x, w_kn, out
    idx = np.sort(rng.choice(nb, size=int(na), replace=False)).astype(np.int32)
    return x, w_kn, idx


def rel_frobenius(y: np.ndarray, y_ref: np.ndarray) -> float:
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    den = np.linalg.norm(y_ref)
    return float(np.linalg.norm(y - y_ref) / den) if den > 0 else float(np.linalg.norm(y - y_ref))


def within_tolerance(y: np.ndarray, y_ref: np.ndarray, rel_fro: float = 1e-3, max_abs_frac: float = 1e-2) -> bool:
    """BASELINE bar for fp16 outputs: relative Frobenius error <= 1e-3 and max-abs error
    <= 1e-2 * max|Y_ref|."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    mx = float(np.max(np.abs(y_ref))) if y_ref.size else 0.0
    return rel_frobenius(y, y_ref) <= rel_fro and float(np.max(np.abs(y - y_ref), initial=0.0)) <= max_abs_frac * mx
