"""Write the golden GEMM / selection fixtures with an implementation that shares nothing with
the oracle: pure-Python float64 loops over the reference's definition
    Y[b, n] = sum_{j in list} sum_{c < 64, 64j+c < K} X[b, 64j+c] * W[n, 64j+c]
(KRN:684-733: one accumulation per list entry; ids past the last block masked out), and a
pure-Python selection by sorting (−sum |x|, id).  Inputs are small and seeded.

    python tests/golden/make_golden.py      # rewrites tests/golden/*.npz
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def gemm_loops(x, w_nk, idx):
    bt, k = x.shape
    n = w_nk.shape[0]
    nblk = (k + 63) // 64
    y = [[0.0] * n for _ in range(bt)]
    for b in range(bt):
        for nn in range(n):
            acc = 0.0
            for j in idx:
                j = int(j)
                if j < 0 or j >= nblk:
                    continue
                for c in range(64):
                    kk = 64 * j + c
                    if kk < k:
                        acc += float(x[b, kk]) * float(w_nk[nn, kk])
            y[b][nn] = acc
    return np.array(y, dtype=np.float64)


def select_loops(x, k):
    bt, kd = x.shape
    nblk = (kd + 63) // 64
    scores = []
    for j in range(nblk):
        s = 0.0
        for b in range(bt):
            for c in range(64):
                kk = 64 * j + c
                if kk < kd:
                    s += abs(float(x[b, kk]))
        scores.append(s)
    order = sorted(range(nblk), key=lambda j: (-scores[j], j))
    return np.array(sorted(order[: min(k, nblk)]), dtype=np.int32), np.array(scores, dtype=np.float64)


CASES = [
    # name, bt, K, N, idx (None = all), seed
    ("gemm_b1_k64_n16_all", 1, 64, 16, None, 1),
    ("gemm_b2_k256_n24_sparse", 2, 256, 24, [3, 0], 2),
    ("gemm_b3_k200_n17_tail", 3, 200, 17, [3, 1], 3),
    ("gemm_b4_k256_n32_dupoor", 4, 256, 32, [2, 2, 9, -1], 4),
    ("gemm_b2_k192_n8_empty", 2, 192, 8, [], 5),
]

SELECT_CASES = [
    ("select_b3_k256", 3, 256, 2, 11),
    ("select_b2_k200_tail", 2, 200, 3, 12),
]


def main():
    for name, bt, k, n, idx, seed in CASES:
        rng = np.random.default_rng(seed)
        x = rng.laplace(0, 0.05, size=(bt, k)).astype(np.float16)
        w = rng.normal(0, 0.02, size=(n, k)).astype(np.float16)
        ids = np.arange((k + 63) // 64, dtype=np.int32) if idx is None else np.array(idx, dtype=np.int32)
        y = gemm_loops(x, w, ids)
        np.savez(os.path.join(HERE, name + ".npz"), x=x, w_nk=w, idx=ids, y=y)
    for name, bt, k, kk, seed in SELECT_CASES:
        rng = np.random.default_rng(seed)
        x = rng.normal(0, 1, size=(bt, k)).astype(np.float16)
        x[:, 64:128] = x[:, 0:64]  # blocks 0 and 1 tie
        sel, scores = select_loops(x, kk)
        np.savez(os.path.join(HERE, name + ".npz"), x=x, k=np.array(kk), sel=sel, scores=scores)


if __name__ == "__main__":
    main()
