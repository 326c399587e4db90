"""Host-side logic of the Python mirror of sampleLogits: option defaults,
history id conversion, the draw-consumption rule, and the workload
generators' algorithmic byte counts (no GPU)."""
import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

from hachiue_amd import sampler, workloads
from hachiue_amd.sampler import _history_ids, draw_rule, resolve_config
from tests import kat


def test_defaults_follow_nullish_coalescing():
    c = resolve_config({})
    assert (c.temperature, c.top_k, c.top_p, c.min_p, c.repetition_penalty) == (0.6, 20, 0.95, 0, 1)
    c = resolve_config({"temperature": 0, "topK": 0, "topP": None, "minP": 0.05})
    assert c.temperature == 0 and c.top_k == 0 and c.top_p == 0.95 and c.min_p == 0.05
    # snake_case field names and unknown GenerateOptions fields
    c = resolve_config({"top_k": 7, "maxNewTokens": 12, "stopTokens": [1]})
    assert c.top_k == 7
    c = resolve_config({"topK": float("inf"), "temperature": float("nan")})
    assert math.isinf(c.top_k) and math.isnan(c.temperature)


def test_history_ids_keep_only_int32_integers():
    ids = _history_ids([0, 5, -1, 2.5, float("nan"), 2**31, 2**31 - 1, 7.0])
    assert ids.tolist() == [0, 5, -1, -1, -1, -1, 2**31 - 1, 7]
    a = np.array([1, 2**40, -3], np.int64)
    assert _history_ids(a).tolist() == [1, -1, -3]


DRAW_CASES = os.path.join(os.path.dirname(__file__), "golden", "draw_cases.json")


def _draw_cases():
    with open(DRAW_CASES) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _draw_cases(), ids=lambda c: c["name"])
def test_draw_rule_hand_cases(case):
    """The decision made before the call, against the hand-derived cases
    (src/sampler.ts:36, :49-69, :76-77, :112)."""
    cfg = resolve_config(kat.config(case["config"]))
    row = kat.f32_array(case["logits"])
    assert draw_rule(cfg, case["vocab"], row, np.array(case["history"], np.int32)) == case["rule"]


def test_draw_rule_without_candidates_outside_the_history():
    NI = -np.inf
    cfg = resolve_config({"temperature": 1.0, "topK": 40, "repetitionPenalty": 1.1})
    row = np.array([1, 2, NI, NI], np.float32)
    # both candidates are in the last 128 entries: only the penalised row tells
    assert draw_rule(cfg, 4, row, np.array([0, 1], np.int32)) == -1
    # id 0 only before the last 128 entries is untouched by the repetition
    # penalty, and with id 2 makes two candidates
    row3 = np.array([1, 2, 3, NI], np.float32)
    assert draw_rule(cfg, 4, row3, np.array([0] + [1] * 128, np.int32)) == 1
    # ... but presence / frequency count the whole history
    pf = resolve_config({"temperature": 1.0, "presencePenalty": 0.5})
    assert draw_rule(pf, 4, row3, np.array([0] + [1] * 128, np.int32)) == -1
    # out-of-range history ids touch nothing
    assert draw_rule(cfg, 4, row, np.array([-1, 4, 99], np.int32)) == 1
    # no penalty: the count is exact
    plain = resolve_config({"temperature": 1.0})
    assert draw_rule(plain, 4, np.array([1, NI, NI, NI], np.float32), np.array([0], np.int32)) == 0
    # fractional topK 1.5 truncates to one slot
    assert draw_rule(resolve_config({"temperature": 1.0, "topK": 1.5}), 4, row, None) == 0


@pytest.mark.skipif(shutil.which("node") is None, reason="node is missing")
def test_js_draw_rule_hand_cases():
    """The JavaScript layer's decision (hachiue_amd/js/index.js drawRule), no GPU."""
    driver = os.path.join(os.path.dirname(__file__), "node", "dropin_check.js")
    out = subprocess.run(["node", driver, "rule", DRAW_CASES], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    got = {r["name"]: r["rule"] for r in map(json.loads, out.stdout.strip().splitlines())}
    for c in _draw_cases():
        assert got[c["name"]] == c["rule"], c["name"]


def test_histories_pack():
    ids, off = sampler._histories([[1, 2], [], [3]], 3)
    assert ids.tolist() == [1, 2, 3] and off.tolist() == [0, 2, 2, 3]
    assert sampler._histories(None, 3) == (None, None)


def test_configs_array():
    arr = sampler.make_configs({"topK": 3}, 4)
    assert len(arr) == 4 and all(c.top_k == 3 for c in arr)
    with pytest.raises(ValueError):
        sampler.make_configs([{}, {}], 3)


def test_workload_shapes_and_bytes():
    wl = workloads.make("headline", 0, rows=2)
    assert wl.logits.shape == (2, workloads.V_QWEN) and wl.logits.dtype == np.float32
    assert wl.algorithmic_bytes() == 2 * (4 * 151936 + 4 * 64 + 4)
    wl = workloads.make("perrow256", 0, rows=3, vocab=5000)
    assert wl.algorithmic_bytes() == 3 * (4 * 5000 + 4 * 1024 + 4)
    wl = workloads.make("gumbel1024", 0, rows=2, vocab=1000)
    assert wl.hist_ids is None and wl.algorithmic_bytes() == 2 * (4 * 1000 + 4)
    assert math.isinf(wl.configs[0]["topK"])
    wl = workloads.make("batch64", 0, rows=2)
    assert wl.algorithmic_bytes() == 2 * (4 * 151936 + 4 * 128 + 4)
    # the headline byte count of the benchmark
    assert workloads.make("headline", 0, rows=1).algorithmic_bytes() * 256 == 155649024
