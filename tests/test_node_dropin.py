"""The JavaScript drop-in (hachiue_amd/js/index.js over the Node-API addon):
loading and error behaviour on the CPU, parity with the oracle on the GPU for
the known answers, row-by-row calls and the (async) batch API."""
import json
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

from hachiue_amd import workloads
from oracle import pyoracle
from tests import kat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tests", "node", "dropin_check.js")
ADDON = os.path.join(ROOT, "hachiue_amd", "node", "hachiue_sampler.node")
NODE = shutil.which("node")
needs_node = pytest.mark.skipif(NODE is None or not os.path.exists(ADDON),
                                reason="node or the addon is missing")


def _node(*args):
    print(f"[node] {' '.join(args[:1])}", flush=True)
    out = subprocess.run([NODE, DRIVER, *args], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-3000:]
    return [json.loads(line) for line in out.stdout.strip().splitlines()]


@needs_node
def test_addon_without_gpu_reports_hip_error():
    from hachiue_amd import hip
    if hip.device_count() > 0:
        pytest.skip("a GPU is visible")
    r = _node("nogpu")[0]
    assert r["vocab0"] == 0            # src/sampler.ts returns 0 without reading a logit
    assert r["error"] == "HS_ERR_HIP"  # no silent CPU fallback
    assert r["type_error"] is True


@needs_node
@pytest.mark.gpu
def test_dropin_known_answers():
    got = {r["name"]: r for r in _node("kat", kat.PATH)}
    for case in kat.cases():
        exp = case["expect"]
        r = got[case["name"]]
        assert r["token"] == exp["token"], case["name"]
        if "logits" in exp:
            assert np.array_equal(np.array(r["logits_bits"], np.uint32),
                                  kat.f32_array(exp["logits"]).view(np.uint32)), case["name"]


def _workload_dir(wl, d):
    import bench
    bench.write_workload_dir(wl, wl.rows, d)


def _oracle(wl):
    ref = wl.logits.copy()
    res = pyoracle.sample_batch(ref, wl.vocab, wl.hist_ids, wl.hist_off, wl.configs, wl.uniforms)
    return res, ref


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", [("headline", dict(rows=6)), ("perrow256", dict(rows=8)),
                                     ("single", dict(greedy=True))])
def test_dropin_rows_match_oracle(name, kw):
    wl = workloads.make(name, 5, **kw)
    with tempfile.TemporaryDirectory() as d:
        _workload_dir(wl, d)
        rows = _node("rows", d)
    res, _ = _oracle(wl)
    for r in range(wl.rows):
        assert rows[r]["token"] == res.token[r] or res.draw_margin[r] < 1e-6, (name, r)


@needs_node
@pytest.mark.gpu
def test_dropin_batch_and_async_match_oracle():
    wl = workloads.make("batch64", 2, rows=16)
    with tempfile.TemporaryDirectory() as d:
        _workload_dir(wl, d)
        out = _node("batch", d)[0]
    res, ref = _oracle(wl)
    ok = (np.array(out["tokens"]) == res.token) | (res.draw_margin < 1e-6)
    assert ok.all()
    assert out["tokens"] == out["tokens_async"]
    assert out["logits_same"]
    assert np.array_equal(np.array(out["penalised"], np.uint32), ref.reshape(-1).view(np.uint32))


@needs_node
def test_greedy_route_decision():
    # src/engine.ts:1600-1601 evaluated by hand on each option object:
    # (temperature ?? 0.6) <= 0 && (repetitionPenalty === undefined || === 1.0)
    want = [False, False, True, True, False, True, False, False, False, False]
    assert _node("route")[0] == want


@needs_node
@pytest.mark.gpu
def test_dropin_argmax_matches_oracle():
    # eight logits of exactly 12.0 per row: the maximum ties, so the WGSL
    # reduction order decides
    wl = workloads.make("headline", 6, rows=8, exact_spikes=True)
    with tempfile.TemporaryDirectory() as d:
        _workload_dir(wl, d)
        out = _node("argmax", d)[0]
    want = pyoracle.wgsl_argmax(wl.logits, wl.vocab).tolist()
    assert out["batch"] == want
    assert out["rows"] == want
    assert out["next"] == want          # nextToken on the greedy route
    assert out["unchanged"]             # the argmax reads the logits only


DRAW_CASES = os.path.join(ROOT, "tests", "golden", "draw_cases.json")


@needs_node
@pytest.mark.gpu
def test_dropin_math_random_calls_follow_the_reference():
    """Math.random() is called exactly when sampleLogits calls it (the
    hand-derived counts of tests/golden/draw_cases.json), row by row and in
    the batch API, and the tokens are the hand-derived ones."""
    with open(DRAW_CASES) as f:
        cases = json.load(f)["cases"]
    out = {r["name"]: r for r in _node("draws", DRAW_CASES)}
    for c in cases:
        assert out[c["name"]]["calls"] == c["calls"], c["name"]
        assert out[c["name"]]["token"] == c["token"], c["name"]
    batch = out["(batch)"]
    assert batch["calls"] == sum(c["calls"] for c in cases)
    assert batch["tokens"] == [c["token"] for c in cases]


@needs_node
@pytest.mark.gpu
def test_dropin_concurrent_calls_on_one_context():
    """Two sampleLogitsBatchAsync calls in flight at once (libuv worker
    threads) and sync sampleLogits calls on the main thread, all on the
    default context: every result equals the oracle's."""
    wl = workloads.make("batch64", 9, rows=12)
    with tempfile.TemporaryDirectory() as d:
        _workload_dir(wl, d)
        out = _node("concurrent", d)[0]
    res, ref = _oracle(wl)
    ok = lambda t: ((np.array(t) == res.token) | (res.draw_margin < 1e-6)).all()
    assert ok(out["a"]) and ok(out["b"]) and ok(out["rows"])
    assert out["b_same"]
    assert np.array_equal(np.array(out["a_bits"], np.uint32), ref.reshape(-1).view(np.uint32))
