"""Shared helpers of the GPU parity tests: seeded inputs on host and device, oracle checks."""
from __future__ import annotations

import numpy as np
import torch

from oracle import bsg_oracle as orc


def to_dev(a: np.ndarray, dev, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def case(seed: int, bt: int, k: int, n: int, na: int, x_dist: str = "laplace"):
    """Seeded BASELINE-style inputs: x [bt,K], w_nk [N,K] (nn.Linear layout), sorted idx."""
    x, w_kn, idx = orc.make_inputs(seed, bt, k, n, x_dist, na=na)
    return x, np.ascontiguousarray(w_kn.T), idx


def assert_close(y: np.ndarray, y_ref: np.ndarray, what: str = "") -> None:
    """BASELINE bar: rel. Frobenius <= 1e-3 and max-abs <= 1e-2 * max|Y_ref| (fp16/bf16 out,
    fp32 accumulation); an all-zero reference requires an all-zero result."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    assert y.shape == y_ref.shape, (y.shape, y_ref.shape)
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    if not np.any(y_ref):
        assert not np.any(y), f"{what}: expected zeros"
        return
    rf = orc.rel_frobenius(y, y_ref)
    ma = float(np.max(np.abs(y - y_ref)))
    mx = float(np.max(np.abs(y_ref)))
    assert rf <= 1e-3 and ma <= 1e-2 * mx, f"{what}: rel_fro={rf:.3e} max_abs={ma:.3e} (max|ref|={mx:.3e})"
