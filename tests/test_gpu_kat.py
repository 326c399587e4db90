"""Every hand-traced known answer of tests/golden/sampler_kat.json through the
device path (hs_sample_batch_device_ex), checked against the expected values
written in the file (not against the oracle): the token, the sorted
candidate ids, the kept-prefix length and the caller's logits after the
in-place penalties (src/sampler.ts:12-118), on every kernel route."""
import numpy as np
import pytest

from tests import kat
from tests.gpu_util import run_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", kat.cases(), ids=lambda c: c["name"])
def test_known_answer_on_device(any_sampler, case):
    logits = kat.f32_array(case["logits"])[None, :]
    before = logits[0].copy()
    vocab = case["vocab"]
    hist = np.asarray(case["history"], np.int64)
    ids = hist.astype(np.int32) if hist.size else np.zeros(1, np.int32)
    off = np.array([0, hist.size], np.int64)
    cfg = kat.config(case["config"])
    cap = max(1, logits.shape[1])
    got = run_gpu(any_sampler, logits, vocab, ids, off, [cfg], [case["u"]], cap,
                  stride=logits.shape[1])
    exp = case["expect"]
    name = case["name"]
    assert int(got.tokens[0]) == exp["token"], name
    if "cand_ids" in exp:
        n = len(exp["cand_ids"])
        assert int(got.n[0]) == n, name
        assert got.cand_ids[0, :n].tolist() == exp["cand_ids"], name
    if "cutoff" in exp:
        assert int(got.cutoff[0]) == exp["cutoff"], name
    if "probs_closed" in exp:
        n = len(exp["probs_closed"])
        np.testing.assert_allclose(got.cand_probs[0, :n].astype(np.float64), exp["probs_closed"],
                                   rtol=1e-6)
    if "logits" in exp:
        assert kat.same_f32(got.logits[0], kat.f32_array(exp["logits"])), name
    if exp.get("logits_closed") == "rep":
        want = kat.rep_closed(before, case["history"], vocab, cfg["repetitionPenalty"])
        assert kat.same_f32(got.logits[0], want), name
