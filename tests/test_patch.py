"""Model-integration host logic without a GPU: the dense-prefill bypass, the lookup-table
nearest row, the module paths and the per-step schedule index (RRD:74-86, 179-203, 342-358)."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from bsa_mi355x import patch


def test_dense_bypass_for_prefill_and_full_density():
    torch.manual_seed(0)
    w = torch.randn(96, 128)
    x = torch.randn(2, 5, 128)  # prefill: 5 tokens per sequence
    stats = {"calls": 0, "wall_s": 0.0}
    cfg = {"best_kern": "naive"}
    y = patch._sparse_linear(x, w, 0.5, cfg, "p", 64, stats, False, None)
    assert torch.equal(y, F.linear(x, w))
    x1 = torch.randn(2, 1, 128)  # decode, but density 1
    assert torch.equal(patch._sparse_linear(x1, w, 1.0, cfg, "p", 64, stats, False, None), F.linear(x1, w))
    assert stats["calls"] == 0


def test_nearest_cfg_and_constants():
    sweep = {"qkvo": {"0.2": {"best_kern": "naive", "best_K": 1}, "0.5": {"best_kern": "bpl", "best_K": 2}}}
    c = patch._nearest_cfg(sweep, "qkvo", 0.41)
    assert c["best_kern"] == "bpl" and c["density_key"] == "0.5"
    c["best_kern"] = "x"  # a copy: the table is untouched
    assert sweep["qkvo"]["0.5"]["best_kern"] == "bpl"
    assert patch._nearest_cfg(sweep, "qkvo", 0.0)["density_key"] == "0.2"
    assert patch.PROJS == ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]
    assert {patch.PROJ_TO_SHAPE[p] for p in patch.PROJS} == {"qkvo", "gate_up", "down"}


class _Layer(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = torch.nn.Module()
        self.mlp = torch.nn.Module()
        for p in patch.PROJS[:4]:
            setattr(self.self_attn, p, torch.nn.Linear(128, 128, bias=False))
        for p in patch.PROJS[4:]:
            setattr(self.mlp, p, torch.nn.Linear(128, 128, bias=False))


def test_get_module_paths():
    model = torch.nn.Module()
    model.model = torch.nn.Module()
    model.model.layers = torch.nn.ModuleList([_Layer(), _Layer()])
    assert patch._get_module(model, 1, "k_proj") is model.model.layers[1].self_attn.k_proj
    assert patch._get_module(model, 0, "down_proj") is model.model.layers[0].mlp.down_proj


def test_step_schedule_skips_the_prefill_entry_and_wraps():
    sweep = {"qkvo": {"0.3": {"best_kern": "naive"}, "0.6": {"best_kern": "bpl"}}}
    state = patch._PatchState(sweep, False, None, 1.0, 0.1, False, None, None, "dense", None, 0.5)
    lin = torch.nn.Linear(128, 128, bias=False)
    fwd = patch._SparseForward(state, lin, 0, "q_proj", 0.9, [0.9, 0.3, 0.6], None, None, lin.forward)
    x_dec = torch.zeros(2, 1, 128)
    got = [fwd._step_density(x_dec) for _ in range(5)]
    assert [d for d, _ in got] == [0.3, 0.6, 0.3, 0.6, 0.3]
    assert [c["best_kern"] for _, c in got] == ["naive", "bpl", "naive", "bpl", "naive"]
    d, c = fwd._step_density(torch.zeros(2, 4, 128))  # prefill keeps the cell's density
    assert d == 0.9 and state.decode_call_counts[(0, "q_proj")] == 5
