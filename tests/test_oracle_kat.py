"""The CPU oracle against the hand-traced known answers of sampler.ts
(tests/golden/sampler_kat.json): both the verbatim O(V*k) replace-min scan
and its heap-ordered equivalent."""
import numpy as np
import pytest

from oracle import pyoracle
from tests import kat

METHODS = [pyoracle.LITERAL, pyoracle.HEAP]


@pytest.mark.parametrize("method", METHODS, ids=["literal", "heap"])
@pytest.mark.parametrize("case", kat.cases(), ids=lambda c: c["name"])
def test_known_answer(case, method):
    logits = kat.f32_array(case["logits"])
    before = logits.copy()
    cfg = kat.config(case["config"])
    exp = case["expect"]
    res = pyoracle.sample_row(logits, case["vocab"], case["history"], cfg, case["u"], method,
                              cap=max(1, len(logits)))
    assert res.token == exp["token"]
    if "cand_ids" in exp:
        assert res.n == len(exp["cand_ids"])
        assert res.cand_ids.tolist() == exp["cand_ids"]
    if "cutoff" in exp:
        assert res.cutoff == exp["cutoff"]
    if "probs_closed" in exp:
        np.testing.assert_allclose(res.cand_probs.astype(np.float64), exp["probs_closed"],
                                   rtol=1e-6)
    if "logits" in exp:
        assert kat.same_f32(logits, kat.f32_array(exp["logits"]))
    if exp.get("logits_closed") == "rep":
        want = kat.rep_closed(before, case["history"], case["vocab"],
                              cfg["repetitionPenalty"])
        assert kat.same_f32(logits, want)


def test_resolve_k_cases():
    d = kat.load()["resolve_k"]
    for top_k, want in d["cases"]:
        assert pyoracle.resolve_k(kat.num(top_k), 100) == want, top_k


def test_defaults():
    d = kat.load()["defaults"]
    r = pyoracle.resolve_config({})
    assert r["temperature"] == d["temperature"]
    assert r["top_k"] == d["topK"]
    assert r["top_p"] == d["topP"]
    assert r["min_p"] == d["minP"]
    assert r["repetition_penalty"] == d["repetitionPenalty"]
    # `??` keeps falsy values: 0 stays 0 (topK 0 later becomes 64, temperature 0 greedy)
    r = pyoracle.resolve_config({"topK": 0, "temperature": 0, "topP": None})
    assert r["top_k"] == 0 and r["temperature"] == 0 and r["top_p"] == 0.95
