"""The Python mirror's stand-in for Math.random() is consumed exactly when
sampleLogits would call Math.random() (hand-derived counts in
tests/golden/draw_cases.json), for single rows and for batches."""
import json
import os
import random

import numpy as np
import pytest

from hachiue_amd import Sampler
from tests import kat

pytestmark = pytest.mark.gpu

PATH = os.path.join(os.path.dirname(__file__), "golden", "draw_cases.json")


def _cases():
    with open(PATH) as f:
        return json.load(f)["cases"]


class _Counter:
    def __init__(self):
        self.calls = 0

    def __call__(self):
        self.calls += 1
        return 0.5


def test_row_draw_counts(sampler, monkeypatch):
    for c in _cases():
        counter = _Counter()
        monkeypatch.setattr(random, "random", counter)
        print(f"[gpu] draw case {c['name']}", flush=True)
        row = kat.f32_array(c["logits"])
        tok = sampler.sample_logits(row, c["vocab"], c["history"], kat.config(c["config"]))
        assert counter.calls == c["calls"], c["name"]
        assert tok == c["token"], c["name"]


def test_batch_draw_counts(sampler, monkeypatch):
    cases = _cases()
    V = max(c["vocab"] for c in cases)
    rows = np.full((len(cases), V), -np.inf, np.float32)
    for r, c in enumerate(cases):
        rows[r, :len(c["logits"])] = kat.f32_array(c["logits"])
    counter = _Counter()
    monkeypatch.setattr(random, "random", counter)
    tok = sampler.sample_logits_batch(rows, V, [c["history"] for c in cases],
                                      [kat.config(c["config"]) for c in cases])
    assert counter.calls == sum(c["calls"] for c in cases)
    assert tok.tolist() == [c["token"] for c in cases]
