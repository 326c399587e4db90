"""The CPU backend of the drop-in (hachiue_amd/js/cpu.js), reached through
createSampler({backend: 'cpu' | 'auto'}): sampleLogits' semantics
(src/sampler.ts:12-118) and the Wasm backend's greedy loop
(src/wasm-backend.ts:1204-1215), against the oracle and hand-derived
answers, and the backend choice of src/engine.ts:626-639.  No GPU."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from hachiue_amd import workloads
from oracle import pyoracle
from tests import kat

NODE = shutil.which("node")
needs_node = pytest.mark.skipif(NODE is None, reason="node is missing")
DRIVER = os.path.join(os.path.dirname(__file__), "node", "dropin_check.js")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
GREEDY_CASES = os.path.join(GOLDEN, "wasm_greedy_cases.json")
DRAW_CASES = os.path.join(GOLDEN, "draw_cases.json")
SPECIAL = {"NaN": np.nan, "Infinity": np.inf, "-Infinity": -np.inf, "-0": -0.0}


def _node(backend, *args):
    env = dict(os.environ)
    if backend:
        env["HS_BACKEND"] = backend
    out = subprocess.run([NODE, DRIVER, *args], capture_output=True, text=True, timeout=600,
                         env=env)
    assert out.returncode == 0, out.stderr[-3000:]
    return [json.loads(line) for line in out.stdout.strip().splitlines()]


def _f32(values):
    return np.array([SPECIAL[v] if isinstance(v, str) else v for v in values], np.float32)


def _greedy_cases():
    with open(GREEDY_CASES) as f:
        return json.load(f)["cases"]


# ---- the oracle's Wasm greedy loop ------------------------------------------

@pytest.mark.parametrize("case", _greedy_cases(), ids=lambda c: c["name"])
def test_oracle_wasm_greedy_hand_cases(case):
    row = _f32(case["logits"])
    assert pyoracle.wasm_greedy(row, case["vocab"])[0] == case["id"]
    # sampleLogits' own greedy branch (a3), which starts from logits[0]
    res = pyoracle.sample_row(row.copy(), case["vocab"], [], {"temperature": 0.0}, 0.5)
    assert res.token == case["a3"]


def test_oracle_wasm_greedy_closed_form():
    """First index of the largest value above -1e30 (compared in binary64),
    0 when none is: numpy's first-occurrence argmax over the admitted values."""
    rng = np.random.default_rng(5)
    pool = np.array([np.nan, -np.inf, np.inf, -0.0, 0.0, -1e30, -2e30, -9.9999e29, 1.0, 2.0, 2.0],
                    np.float32)
    for _ in range(400):
        V = int(rng.integers(1, 40))
        row = rng.choice(pool, V) if rng.random() < 0.7 else np.round(rng.standard_normal(V) * 2)
        row = np.asarray(row, np.float32)
        x = row.astype(np.float64)
        ok = ~np.isnan(x) & (x > -1e30)
        want = 0
        if ok.any():
            m = x[ok].max()
            want = int(np.flatnonzero(ok & (x == m))[0])
        assert pyoracle.wasm_greedy(row, V)[0] == want, row


# ---- the CPU backend ---------------------------------------------------------

@needs_node
@pytest.mark.parametrize("backend", ["cpu", "auto"])
def test_backend_choice(backend):
    from hachiue_amd import hip
    if hip.device_count() > 0:
        pytest.skip("a GPU is visible: 'auto' takes the HIP backend")
    r = _node(None, "backend", backend)[0]
    assert r["info"]["backend"] == "cpu" and r["token"] == 1
    if backend == "auto":
        assert "fallbackReason" in r["info"] and r["info"]["fallbackReason"]
    else:
        assert "fallbackReason" not in r["info"]


@needs_node
def test_backend_choice_refusals():
    from hachiue_amd import hip
    assert _node(None, "backend", "bogus")[0]["error"] == "TypeError"
    if hip.device_count() == 0:
        # 'hip' (the default) never falls back
        assert _node(None, "backend", "hip")[0]["error"] == "HS_ERR_HIP"


@needs_node
def test_cpu_known_answers():
    got = {r["name"]: r for r in _node("cpu", "kat", kat.PATH)}
    for case in kat.cases():
        exp = case["expect"]
        r = got[case["name"]]
        assert r["token"] == exp["token"], case["name"]
        if "logits" in exp:
            assert np.array_equal(np.array(r["logits_bits"], np.uint32),
                                  kat.f32_array(exp["logits"]).view(np.uint32)), case["name"]


@needs_node
def test_cpu_draw_consumption():
    """Math.random() is called exactly when the reference calls it, row by
    row and across a batch (hand-derived cases)."""
    with open(DRAW_CASES) as f:
        cases = json.load(f)["cases"]
    out = {r["name"]: r for r in _node("cpu", "draws", DRAW_CASES)}
    for c in cases:
        assert out[c["name"]]["calls"] == c["calls"], c["name"]
        assert out[c["name"]]["token"] == c["token"], c["name"]
    batch = out["(batch)"]
    assert batch["calls"] == sum(c["calls"] for c in cases)
    assert batch["tokens"] == [c["token"] for c in cases]


@needs_node
def test_cpu_greedy_route_hand_cases():
    got = {r["name"]: r for r in _node("cpu", "greedy", GREEDY_CASES)}
    for c in _greedy_cases():
        r = got[c["name"]]
        assert r["id"] == c["id"] and r["batch"] == c["id"] and r["next"] == c["id"], c["name"]
        assert r["unchanged"], c["name"]


def _adversarial(seed=11, V=3000):
    """Rows the reference's semantics single out: ties at and inside the top
    k, NaN / +-Infinity / -0, k beyond the finite count, fractional / zero /
    negative / infinite topK, NaN options, penalties on edge ids."""
    r = np.random.default_rng(seed)
    rows, cfgs, hists = [], [], []

    def add(row, cfg, hist=()):
        rows.append(np.asarray(row, np.float32))
        cfgs.append(cfg)
        hists.append(np.asarray(hist, np.int32))

    base = (r.standard_normal(V) * 2).astype(np.float32)
    coarse = np.round(r.standard_normal(V) * 3).astype(np.float32)
    special = base.copy()
    special[r.choice(V, 40, replace=False)] = np.nan
    special[r.choice(V, 40, replace=False)] = -np.inf
    special[[5, 6]] = [-0.0, 0.0]
    inf = base.copy(); inf[[100, 900]] = np.inf
    sparse = np.full(V, -np.inf, np.float32); sparse[[3, 9, 11, 30]] = [1.0, 2.0, 1.0, 2.0]
    s = dict(temperature=0.8, topK=40, topP=0.9)
    add(base, s)
    add(coarse, dict(temperature=1.3, topK=64, topP=1.0))
    add(coarse, dict(temperature=1.3, topK=700, topP=0.97))
    add(coarse, dict(temperature=1.0, topK=float("inf"), topP=0.9))
    add(special, s, [5, 6, 7, -1, V, 2**31 - 1])
    add(special, dict(repetitionPenalty=1.4, **s), [5, 6, 7, 7, -1, V])
    add(inf, dict(temperature=1.0, topK=10, topP=1.0))
    add(sparse, dict(temperature=1.0, topK=40))
    add(sparse, dict(temperature=1.0, topK=2.7, topP=1.0))
    add(base, dict(temperature=1.0, topK=0))
    add(base, dict(temperature=1.0, topK=-3))
    add(base, dict(temperature=float("nan"), topK=40))
    add(base, dict(temperature=1.0, topK=40, topP=float("nan"), minP=float("nan")))
    add(base, dict(temperature=0.5, topK=40, minP=0.2))
    add(base, dict(temperature=0.0, repetitionPenalty=1.5), list(r.integers(0, V, 300)))
    add(base, dict(repetitionPenalty=0.7, presencePenalty=0.4, frequencyPenalty=0.1, **s),
        list(r.integers(0, 60, 500)))
    add(base, dict(presencePenalty=-1.0, **s), [0, 0, V - 1])
    add(np.full(V, np.nan, np.float32), s)
    add(np.ones(V, np.float32), dict(temperature=1.0, topK=1000, topP=0.5))
    off = np.zeros(len(rows) + 1, np.int64)
    for i, h in enumerate(hists):
        off[i + 1] = off[i] + h.size
    ids = np.concatenate(hists).astype(np.int32)
    us = r.random(len(rows))
    us[0] = 0.0
    return workloads.Workload("adversarial", np.stack(rows), V, ids, off, cfgs, us)


def _check_against_oracle(wl, tmp_path, mode):
    import bench
    d = str(tmp_path / f"{wl.name}_{mode}")
    bench.write_workload_dir(wl, wl.rows, d)
    ref = wl.logits.copy()
    want = pyoracle.sample_batch(ref, wl.vocab, wl.hist_ids, wl.hist_off, wl.configs, wl.uniforms)
    out = _node("cpu", mode, d)
    if mode == "rows":
        got = [r["token"] for r in out]
    else:
        got = out[0]["tokens"]
        assert out[0]["tokens_async"] == got
        pen = np.array(out[0]["penalised"], np.uint32).reshape(ref.shape)
        assert np.array_equal(pen, ref.view(np.uint32)), "penalised logits"
    assert got == [int(t) for t in want.token], wl.name


@needs_node
@pytest.mark.parametrize("mode", ["rows", "batch"])
def test_cpu_matches_oracle_adversarial(tmp_path, mode):
    _check_against_oracle(_adversarial(), tmp_path, mode)


@needs_node
@pytest.mark.parametrize("name,rows,vocab", [("headline", 6, None), ("perrow256", 10, None),
                                             ("gumbel1024", 3, 20000), ("v262k512", 2, None)])
def test_cpu_matches_oracle_workloads(tmp_path, name, rows, vocab):
    kw = dict(rows=rows)
    if vocab:
        kw["vocab"] = vocab
    _check_against_oracle(workloads.make(name, 0, **kw), tmp_path, "batch")


@needs_node
@pytest.mark.parametrize("name", ["adversarial", "perrow256", "gumbel1024"])
def test_cpu_candidates_match_oracle(tmp_path, name):
    """Candidate ids in order, probabilities bit for bit, and the cutoff."""
    import bench
    wl = _adversarial() if name == "adversarial" else workloads.make(
        name, 1, rows=4, vocab=12000 if name == "gumbel1024" else None)
    d = str(tmp_path / name)
    bench.write_workload_dir(wl, wl.rows, d)
    got = _node(None, "cpu-candidates", d)
    for r in range(wl.rows):
        row = wl.logits[r].copy()
        cfg = wl.configs[r]
        want = pyoracle.sample_row(row, wl.vocab, wl.history(r), cfg, float(wl.uniforms[r]))
        g = got[r]
        assert g["token"] == want.token, (name, r)
        if pyoracle.resolve_config(cfg)["temperature"] <= 0:
            continue
        assert g["ids"] == want.cand_ids.tolist(), (name, r)
        if want.n >= 2:
            assert g["probs"] == want.cand_probs.view(np.uint32).tolist(), (name, r)
            assert g["cutoff"] == want.cutoff, (name, r)


@needs_node
@pytest.mark.gpu
def test_cpu_and_hip_backends_agree(tmp_path):
    """On a GPU host 'auto' takes HIP, and both backends give the same tokens."""
    import bench
    r = _node(None, "backend", "auto")[0]
    assert r["info"]["backend"] == "hip" and "fallbackReason" not in r["info"]
    wl = workloads.make("headline", 2, rows=16)
    d = str(tmp_path / "headline")
    bench.write_workload_dir(wl, wl.rows, d)
    cpu = [x["token"] for x in _node("cpu", "rows", d)]
    hip = [x["token"] for x in _node("hip", "rows", d)]
    assert cpu == hip
