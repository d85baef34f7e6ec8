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


def test_decode_step_full_32_layers(dev):
    """BASELINE config 5 at its real size: 32 layers x {qkv, o, gate/up, down}, B=64, density
    0.48, ~13 GB of packed weights, captured as one graph.  Every projection's selected blocks
    are bit-exact vs the oracle (all 128), the first and last layer's outputs are within the
    BASELINE tolerance, and three replays equal the eager step bit for bit."""
    step = DecodeStep(batch=64, density=0.48, n_layers=32, device=dev)
    assert step.resident_weight_bytes == 32 * (64 * 64 * (12288 + 4096 + 22016) + 172 * 64 * 4096) * 2
    step.run()
    torch.cuda.synchronize()
    eager = [p.y.clone() for _, p in step.projections()]
    for li, p in step.projections():
        x = p.x.cpu().numpy()
        want = orc.select_topk_l1(x, p.keep)
        assert np.array_equal(p.idx[: len(want)].cpu().numpy(), want), (li, p.name)
        assert int(p.cnt.item()) == len(want), (li, p.name)
        if li in (0, 31):
            w_nk = np.ascontiguousarray(orc.tile_unpermute(p.packed.cpu().numpy(), p.n).reshape(-1, p.n)[: p.k].T)
            assert_close(p.y.float().cpu().numpy(), orc.gemm_ref(x, w_nk, want), f"layer {li} {p.name}")
    step.capture()
    for r in range(3):
        for _, p in step.projections():
            p.y.fill_(float("nan"))
            p.idx.fill_(-1)
        torch.cuda.synchronize()
        step.replay()
        torch.cuda.synchronize()
        for (li, p), e in zip(step.projections(), eager):
            assert torch.equal(p.y.view(torch.int16), e.view(torch.int16)), (r, li, p.name)
            want = orc.select_topk_l1(p.x.cpu().numpy(), p.keep) if li in (0, 31) else None
            if want is not None:
                assert np.array_equal(p.idx[: len(want)].cpu().numpy(), want), (r, li, p.name)
    assert step.active_bytes == 32 * (31 * 64 * 12288 + 31 * 64 * 4096 + 31 * 64 * 22016 + 83 * 64 * 4096) * 2
    del step, eager
    torch.cuda.empty_cache()
