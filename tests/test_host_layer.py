"""Host-side logic of the Python mirror of sampleLogits: option defaults,
history id conversion, the draw-consumption rule, and the workload
generators' algorithmic byte counts (no GPU)."""
import math

import numpy as np
import pytest

from hachiue_amd import sampler, workloads
from hachiue_amd.sampler import _history_ids, _may_draw, resolve_config


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


def test_draw_only_when_the_reference_draws():
    assert not _may_draw(resolve_config({"temperature": 0}), 100)
    assert not _may_draw(resolve_config({"temperature": -1}), 100)
    assert not _may_draw(resolve_config({"temperature": float("nan"), "topK": 1}), 100)
    assert not _may_draw(resolve_config({"topK": 1}), 100)
    assert not _may_draw(resolve_config({"topK": 40}), 1)
    assert _may_draw(resolve_config({"topK": 40}), 100)
    assert _may_draw(resolve_config({"topK": 0}), 100)     # 0 -> 64


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
