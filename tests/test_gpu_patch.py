"""End-to-end model integration on the GPU: a small random-init Llama (transformers, built from
a config, no download) patched with `_patch_roundrobin_sparse`.  Prefill must be the dense
model bit for bit; every decode-time projection must match the oracle on its own input (the
reference's selector rules, then the block-sparse product); the energy gate, mask reuse, step
schedules and `_restore` behave as in RRD:287-508."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from bsa_mi355x import patch
from bsa_mi355x.select import _energy_expanded_active_blocks
from helpers import assert_close
from oracle import bsg_oracle as orc

pytestmark = pytest.mark.gpu

SWEEP = {shape: {"0.3": {"best_kern": "naive", "best_K": 1, "best_tile": None},
                 "0.5": {"best_kern": "bpl", "best_K": 1, "best_tile": None},
                 "0.7": {"best_kern": "naive", "best_K": 2, "best_tile": [16, 64, 2, 3]},
                 "0.9": {"best_kern": "bpl", "best_K": 2, "best_tile": [16, 64, 2, 3]}}
         for shape in ("qkvo", "gate_up", "down")}


@pytest.fixture(scope="module")
def model(dev):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(1234)
    cfg = transformers.LlamaConfig(hidden_size=256, intermediate_size=704, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=4, vocab_size=512,
                                   max_position_embeddings=128)
    m = transformers.LlamaForCausalLM(cfg).to(device=dev, dtype=torch.float16).eval()
    return m


def _alloc(m, density):
    return {str(li): {p: density for p in patch.PROJS} for li in range(len(m.model.layers))}


def _capture(m):
    """Forward hooks recording (input, output) of every projection."""
    rec, hooks = [], []
    for li in range(len(m.model.layers)):
        for p in patch.PROJS:
            mod = patch._get_module(m, li, p)
            hooks.append(mod.register_forward_hook(
                lambda mod, inp, out, li=li, p=p: rec.append((li, p, inp[0].detach().clone(), out.detach().clone()))))
    return rec, hooks


def _decode(m, ids, steps):
    with torch.inference_mode():
        out = m(input_ids=ids, use_cache=True, return_dict=False)
        logits, past = out[0], out[1]
        nxt = logits[:, -1:].argmax(-1)
        for _ in range(steps):
            out = m(input_ids=nxt, past_key_values=past, use_cache=True, return_dict=False)
            past = out[1]
            nxt = out[0][:, -1:].argmax(-1)
    return logits


def _oracle(x, w, density, fixed=None):
    x2 = x.reshape(-1, x.shape[-1]).float().cpu().numpy().astype(np.float16)
    wn = w.detach().float().cpu().numpy().astype(np.float16)
    if fixed is None:
        nb = x2.shape[1] // 64
        fixed, _, _ = orc.select_scored_ref(x2, orc.n_keep(density, nb), score="l2_mean")
    return orc.gemm_ref(x2, wn, fixed)


def test_prefill_is_dense_and_decode_matches_oracle(dev, model):
    m = model
    ids = torch.randint(0, 512, (4, 6), device=dev)
    dense = _decode(m, ids, 0)
    originals, stats = patch._patch_roundrobin_sparse(m, _alloc(m, 0.5), SWEEP, False)
    try:
        rec, hooks = _capture(m)
        sparse = _decode(m, ids, 2)
        for h in hooks:
            h.remove()
    finally:
        patch._restore(originals)
    assert torch.equal(dense, sparse), "prefill must run the dense linears"
    dec = [r for r in rec if r[2].shape[1] == 1]
    assert len(dec) == 2 * 2 * 7 and stats["calls"] == len(dec)
    for li, p, x, y in dec:
        w = patch._get_module(m, li, p).weight
        assert_close(y.reshape(-1, y.shape[-1]).float().cpu().numpy(), _oracle(x, w, 0.5), f"decode L{li} {p}")
    # after _restore every call is dense again
    rec, hooks = _capture(m)
    _decode(m, ids, 1)
    for h in hooks:
        h.remove()
    for li, p, x, y in rec:
        assert torch.equal(y, F.linear(x, patch._get_module(m, li, p).weight.detach()))


@pytest.mark.parametrize("density", [0.3, 0.7, 0.9])
def test_each_lookup_row_kernel(dev, model, density):
    """naive / bpl, with and without split-K, as the nearest lookup row names them."""
    m = model
    originals, _ = patch._patch_roundrobin_sparse(m, _alloc(m, density), SWEEP, True)
    try:
        rec, hooks = _capture(m)
        _decode(m, torch.randint(0, 512, (3, 4), device=dev), 1)
        for h in hooks:
            h.remove()
    finally:
        patch._restore(originals)
    for li, p, x, y in [r for r in rec if r[2].shape[1] == 1]:
        w = patch._get_module(m, li, p).weight
        assert_close(y.reshape(-1, y.shape[-1]).float().cpu().numpy(), _oracle(x, w, density), f"{density} {p}")


@pytest.mark.parametrize("mode", ["dense", "expand", "scaled"])
def test_energy_gate_modes(dev, model, mode):
    m = model
    originals, stats = patch._patch_roundrobin_sparse(m, _alloc(m, 0.3), SWEEP, False, energy_gate_keep=0.999,
                                                      energy_gate_mode=mode)
    try:
        rec, hooks = _capture(m)
        _decode(m, torch.randint(0, 512, (2, 4), device=dev), 1)
        for h in hooks:
            h.remove()
    finally:
        patch._restore(originals)
    dec = [r for r in rec if r[2].shape[1] == 1]
    # the gate is checked on every call, as in RRD:360-368; a prefill call's ratio is 1.0
    # (RRD:125-126), so only the decode calls fall back
    assert stats["energy_gate_checks"] == len(rec)
    cells = stats["cell_energy_stats"]
    assert len(cells) == 2 * 7 and all(c["checks"] == 2 for c in cells.values())
    for li, p, x, y in dec:
        w = patch._get_module(m, li, p).weight
        yv = y.reshape(-1, y.shape[-1]).float().cpu().numpy()
        if mode == "dense":
            assert torch.equal(y, F.linear(x, w.detach()))
        elif mode == "expand":
            active, _, _ = _energy_expanded_active_blocks(x, 0.3, 64, 0.999)
            assert_close(yv, _oracle(x, w, None, fixed=active.cpu().numpy()), f"expand {p}")
        else:
            # sparsity 0.7 scaled by 0.5 -> density 0.65, the 0.7 row's kernel
            assert_close(yv, _oracle(x, w, 0.65), f"scaled {p}")
    key = {"dense": "energy_gate_dense_fallbacks", "expand": "energy_gate_expands",
           "scaled": "energy_gate_scaled_fallbacks"}[mode]
    assert stats[key] == len(dec)


def test_mask_reuse_and_step_schedule(dev, model):
    m = model
    sched = {(li, p): [1.0, 0.3, 0.7] for li in range(2) for p in patch.PROJS}
    originals, stats = patch._patch_roundrobin_sparse(m, _alloc(m, 0.5), SWEEP, False, step_density_alloc=sched)
    try:
        rec, hooks = _capture(m)
        _decode(m, torch.randint(0, 512, (2, 4), device=dev), 3)
        for h in hooks:
            h.remove()
    finally:
        patch._restore(originals)
    dec = [r for r in rec if r[2].shape[1] == 1]
    assert len(dec) == 3 * 14
    for i, (li, p, x, y) in enumerate(dec):
        d = [0.3, 0.7, 0.3][i // 14]
        w = patch._get_module(m, li, p).weight
        assert_close(y.reshape(-1, y.shape[-1]).float().cpu().numpy(), _oracle(x, w, d), f"step {i // 14} {p}")
    # reuse: the second decode call of a cell runs on the first call's mask
    originals, stats = patch._patch_roundrobin_sparse(m, _alloc(m, 0.5), SWEEP, False, reuse_masks=True)
    try:
        rec, hooks = _capture(m)
        _decode(m, torch.randint(0, 512, (2, 4), device=dev), 2)
        for h in hooks:
            h.remove()
    finally:
        patch._restore(originals)
    dec = [r for r in rec if r[2].shape[1] == 1]
    first = {(li, p): x for li, p, x, _ in dec[:14]}
    for li, p, x, y in dec[14:]:
        w = patch._get_module(m, li, p).weight
        x0 = first[(li, p)].reshape(-1, x.shape[-1]).float().cpu().numpy().astype(np.float16)
        mask, _, _ = orc.select_scored_ref(x0, orc.n_keep(0.5, x0.shape[1] // 64), score="l2_mean")
        assert_close(y.reshape(-1, y.shape[-1]).float().cpu().numpy(), _oracle(x, w, None, fixed=mask),
                     f"reuse {p}")


def test_patched_linear_call_site_follows_input_prior_and_weight_updates(dev):
    """A decode call site of the patched linear resolves its library call once; later calls
    with new activations, an in-place prior update, an in-place weight update and a different
    scale tensor must each give the reference's selection and product (oracle, float64 rules)."""
    bt, k, n, density = 16, 4096, 1024, 0.4
    rng = np.random.default_rng(41)
    w = torch.from_numpy(rng.normal(0, 0.02, size=(n, k)).astype(np.float16)).to(dev)
    prior = torch.from_numpy(rng.uniform(0, 1, size=k // 64).astype(np.float32)).to(dev)
    cfg = {"best_kern": "naive", "best_K": 1, "best_tile": None}
    stats = {"calls": 0, "wall_s": 0.0}
    nk = orc.n_keep(density, k // 64)

    def call(x, scale=None):
        xt = torch.from_numpy(x).to(dev).view(bt, 1, k)
        out = patch._sparse_linear(xt, w, density, cfg, "prep_linear", 64, stats, False, None, block_prior=prior,
                                   prior_alpha=0.7, prior_eps=0.1, block_score_scale=scale)
        torch.cuda.synchronize()
        return out.view(bt, n).float().cpu().numpy()

    def want(x, scale=None):
        ids, _, _ = orc.select_scored_ref(x, nk, "energy" if scale is not None else "l2_mean",
                                          prior=prior.cpu().numpy(), alpha=0.7, eps=0.1,
                                          scale=None if scale is None else scale.cpu().numpy())
        return orc.gemm_ref(x, w.cpu().numpy(), ids)

    for step in range(3):
        x = rng.normal(0, 1, size=(bt, k)).astype(np.float16)
        assert_close(call(x), want(x), f"step {step}")
    prior.copy_(torch.linspace(2.0, 0.0, k // 64, device=dev))
    x = rng.normal(0, 1, size=(bt, k)).astype(np.float16)
    assert_close(call(x), want(x), "after an in-place prior update")
    with torch.no_grad():
        w.mul_(-1.0)
    assert_close(call(x), want(x), "after an in-place weight update")
    scale = torch.from_numpy(rng.uniform(0.5, 2.0, size=k).astype(np.float32)).to(dev)
    assert_close(call(x, scale), want(x, scale), "with a channel scale")
    assert stats["calls"] == 6
