"""Decode-step graph (two layers here): every projection's selected blocks are
bit-exact vs the oracle, every output is within the BASELINE tolerance, and graph replays equal
the eager step bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from bsa_mi355x.decode import DecodeStep
from helpers import assert_close
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu


def test_decode_step_two_layers(dev):
    step = DecodeStep(batch=64, density=0.48, n_layers=2, device=dev)
    step.run()
    torch.cuda.synchronize()
    eager = [p.y.clone() for _, p in step.projections()]
    for li, p in step.projections():
        x = p.x.cpu().numpy()
        want = orc.select_topk_l1(x, p.keep)
        assert np.array_equal(p.idx[: len(want)].cpu().numpy(), want), (li, p.name)
        assert int(p.cnt.item()) == len(want)
        w_nk = np.ascontiguousarray(orc.tile_unpermute(p.packed.cpu().numpy(), p.n).reshape(-1, p.n)[: p.k].T)
        assert_close(p.y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), f"layer {li} {p.name}")
    step.capture()
    for r in range(3):
        for _, p in step.projections():
            p.y.fill_(float("nan"))
        torch.cuda.synchronize()
        step.replay()
        torch.cuda.synchronize()
        for (li, p), e in zip(step.projections(), eager):
            assert torch.equal(p.y.view(torch.int16), e.view(torch.int16)), (r, li, p.name)
    assert step.active_bytes == 2 * (31 * 64 * 12288 + 31 * 64 * 4096 + 31 * 64 * 22016 + 83 * 64 * 4096) * 2
