"""The JavaScript restatement of sampler.ts (oracle/sampler_port.js, the CPU
baseline run under Node) against the hand-traced known answers, and against
the C oracle on seeded workloads: two independent restatements must agree
bit for bit (tokens, candidate order, float32 probabilities)."""
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
DRIVER = os.path.join(ROOT, "oracle", "cpu_bench.js")
NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _node(*args):
    out = subprocess.run([NODE, DRIVER, *args], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    return [json.loads(line) for line in out.stdout.strip().splitlines()]


def test_port_known_answers():
    got = {r["name"]: r for r in _node("kat", kat.PATH)}
    for case in kat.cases():
        r = got[case["name"]]
        exp = case["expect"]
        assert r["token"] == exp["token"], case["name"]
        if "cand_ids" in exp:
            assert r["ids"] == exp["cand_ids"], case["name"]
        if "cutoff" in exp:
            assert r["cutoff"] == exp["cutoff"], case["name"]
        if "probs_closed" in exp:
            np.testing.assert_allclose(r["probs"], exp["probs_closed"], rtol=1e-6)
        if "logits" in exp:
            bits = np.array(r["logits_bits"], np.uint32)
            assert np.array_equal(bits, kat.f32_array(exp["logits"]).view(np.uint32)), case["name"]


@pytest.mark.parametrize("name,kw", [
    ("headline", dict(rows=8)),
    ("perrow256", dict(rows=12, vocab=30000)),
    ("v262k512", dict(rows=4, vocab=40000)),
    ("batch64", dict(rows=6)),
    ("single", dict(exact_spikes=True)),
])
def test_port_matches_c_oracle(name, kw):
    import bench
    wl = workloads.make(name, 3, **kw)
    with tempfile.TemporaryDirectory() as d:
        bench.write_workload_dir(wl, wl.rows, d)
        js = _node("check", d, "64")
    ref = wl.logits.copy()
    res = pyoracle.sample_batch(ref, wl.vocab, wl.hist_ids, wl.hist_off, wl.configs, wl.uniforms,
                                pyoracle.HEAP, 64)
    for r in range(wl.rows):
        assert js[r]["token"] == res.token[r], (name, r)
        n = min(int(res.n[r]), 64)
        assert js[r]["ids"][:n] == res.cand_ids[r, :n].tolist(), (name, r)
        assert np.array_equal(np.float32(js[r]["probs"][:n]).view(np.uint32),
                              res.cand_probs[r, :n].view(np.uint32)), (name, r)
