"""hs_sample_batch_device_noalloc (the entry point that allocates nothing:
its workspace is the GPU's static scratch array) against
hs_sample_batch_device on the same inputs: identical tokens and penalised
logits, on calls in a row whose second is smaller (the scratch keeps the
first call's contents), and an upload-free repeat of the second."""
import numpy as np
import pytest

from hachiue_amd import hip, workloads
from hachiue_amd.sampler import SamplerError, make_configs

pytestmark = pytest.mark.gpu

# one config per kernel route: row kernel (k <= 64), mid kernel (64 < k <=
# 1024), large-k kernel, penalty pre-pass (presence / frequency), greedy
MIX = [dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
       dict(temperature=0.9, topK=300, topP=0.95),
       dict(temperature=1.0, topK=5000, topP=0.9),
       dict(temperature=0.8, topK=100, topP=0.9, presencePenalty=0.4, frequencyPenalty=0.2),
       dict(temperature=0.0, repetitionPenalty=1.3)]


def _inputs(rows, vocab, seed, configs):
    wl = workloads.make("headline", seed, rows=rows, vocab=vocab)
    return wl.logits, wl.hist_ids, wl.hist_off, wl.uniforms, configs


def _run(sampler, noalloc, logits, ids, off, u, configs):
    rows, vocab = logits.shape
    d_l = hip.DeviceArray.from_numpy(logits)
    d_i = hip.DeviceArray.from_numpy(ids)
    d_o = hip.DeviceArray.from_numpy(off)
    d_u = hip.DeviceArray.from_numpy(u)
    d_t = hip.DeviceArray(rows, np.int32)
    cfgs = make_configs(configs, rows)
    fn = sampler.sample_device_noalloc if noalloc else sampler.sample_device
    fn(d_l.addr, rows, vocab, vocab, d_i.addr, d_o.addr, cfgs, d_u.addr, d_t.addr)
    hip.synchronize()
    return d_t.download(), d_l.download()


def test_noalloc_matches_the_allocating_entry_point(sampler):
    calls = [(300, 151936, 1, [MIX[r % len(MIX)] for r in range(300)]),
             (3, 151936, 2, [MIX[0]] * 3),          # split rows: 9 parts each
             (3, 151936, 2, [MIX[0]] * 3),          # same configs: no upload
             (40, 50000, 3, [MIX[(r * 7) % len(MIX)] for r in range(40)])]
    for rows, vocab, seed, configs in calls:
        print(f"[gpu] noalloc rows={rows} vocab={vocab} seed={seed}", flush=True)
        logits, ids, off, u, cfg = _inputs(rows, vocab, seed, configs)
        want_t, want_l = _run(sampler, False, logits, ids, off, u, cfg)
        got_t, got_l = _run(sampler, True, logits, ids, off, u, cfg)
        assert np.array_equal(got_t, want_t), (rows, vocab)
        assert np.array_equal(got_l.view(np.uint32), want_l.view(np.uint32)), (rows, vocab)


def test_noalloc_limits(sampler):
    d_t = hip.DeviceArray(2049, np.int32)
    d_u = hip.DeviceArray(2049, np.float64)
    with pytest.raises(SamplerError) as e:
        sampler.sample_device_noalloc(d_t.addr, 2049, 8, 8, None, None, {}, d_u.addr, d_t.addr)
    assert e.value.status == 4 and "2048" in str(e.value)
    with pytest.raises(SamplerError) as e:
        sampler.sample_device_noalloc(d_t.addr, 1, 1 << 20, 1 << 20, None, None, {}, d_u.addr,
                                      d_t.addr)
    assert e.value.status == 4
