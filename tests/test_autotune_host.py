"""First-call tuning bookkeeping on the host (no GPU): keys, the persisted cache, and that a
tabulated problem never reaches the tuner."""
from __future__ import annotations

import json

import pytest

from bsa_mi355x import autotune, tuning
from bsa_mi355x._lib import Plan


@pytest.fixture
def fresh(tmp_path):
    saved = dict(autotune._STATE)
    autotune.clear()
    yield tmp_path
    autotune.clear()
    autotune._STATE.clear()
    autotune._STATE.update(saved)


def test_key_names_the_reference_autotune_key_plus_source_and_dtype(fresh):
    # KRN:684-687 keys on (N_OUT, M, BATCHSIZE, NUM_ACTIVE_BLOCKS)
    k = autotune.key(1000, 32, 5, 7, "list", 0)
    assert k == (1000, 32, 5, 7, "list", 0)
    assert autotune.key(1000, 32, 5, 7, "bitmap", 0) != k
    assert autotune.key(1000, 32, 5, 7, "list", 1) != k


def test_cache_persists_and_reloads(fresh):
    path = str(fresh / "tuned.json")
    autotune.set_autotune(True, cache_path=path)
    k = autotune.key(1000, 32, 5, 7, "list", 0)
    assert autotune.cached(k) is None
    autotune.record(k, Plan(2, 16, 4, 4, 16, 1), 12.5)
    with open(path) as f:
        data = json.load(f)
    assert data["entries"] == [{"key": [1000, 32, 5, 7, "list", 0], "plan": [2, 16, 4, 4, 16, 1], "us": 12.5}]
    autotune.clear()
    autotune.set_autotune(True, cache_path=path)  # reload from the file
    assert autotune.cached(k).as_tuple() == (2, 16, 4, 4, 16, 1)
    assert autotune.stats()["keys"] == 1


def test_tabulated_shapes_are_not_tuned():
    # the shipped table covers the Llama-2-7B shapes: lookup answers, so the tuner is never asked
    assert tuning.lookup(16, 4096, 172, 86) is not None
    assert tuning.lookup(16, 1000, 32, 7) is None


def test_tune_picks_the_fastest_runnable_candidate(fresh, monkeypatch):
    """tune() with a fake launcher and fake timings: rejected candidates are skipped and the
    finalist with the lowest median wins."""
    import torch

    speed = {(1, 16, 4, 4, 16, 1): 9.0, (2, 16, 4, 4, 16, 1): 7.0, (1, 16, 2, 4, 16, 1): 8.0}
    rejected = (4, 16, 8, 4, 16, 1)
    clock = {"ms": 0.0}  # device time: every accepted launch advances it by its plan's µs

    def launch(p):
        if p.as_tuple() == rejected:
            return -5
        clock["ms"] += speed[p.as_tuple()] / 1000.0
        return 0

    class FakeEvent:
        def __init__(self, enable_timing=True):
            self.t = 0.0

        def record(self, stream=None):
            self.t = clock["ms"]

        def synchronize(self):
            pass

        def elapsed_time(self, other):
            return other.t - self.t

    class FakeStream:
        pass

    monkeypatch.setattr(torch.cuda, "Event", FakeEvent)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: FakeStream())
    k = autotune.key(1000, 32, 5, 7, "list", 0)
    cands = [Plan(*t) for t in list(speed) + [rejected]]
    best = autotune.tune(k, cands, launch, device=None, reps=1, finalists=3, final_reps=1)
    assert best.as_tuple() == (2, 16, 4, 4, 16, 1)
    assert autotune.cached(k).as_tuple() == (2, 16, 4, 4, 16, 1)
    assert autotune.stats()["tunes"] == 1
