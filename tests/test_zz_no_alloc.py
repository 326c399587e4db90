"""hs_sample_batch_device_noalloc (the entry point that allocates nothing:
its workspace is the GPU's static scratch array) against
hs_sample_batch_device and the oracle on the same inputs: identical tokens
and penalised logits, on calls in a row whose second is smaller (the scratch
keeps the first call's contents), an upload-free repeat of the second, and
large-k rows whose ties are replayed in the scratch's slot region.  A call
on a stream under graph capture is refused before anything is enqueued."""
import ctypes

import numpy as np
import pytest

from hachiue_amd import hip, workloads
from hachiue_amd.sampler import SamplerError, make_configs
from oracle import pyoracle

pytestmark = pytest.mark.gpu

# one config per kernel route: row kernel (k <= 64), mid kernel (64 < k <=
# 1024), large-k kernel, penalty pre-pass (presence / frequency), greedy
MIX = [dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
       dict(temperature=0.9, topK=300, topP=0.95),
       dict(temperature=1.0, topK=5000, topP=0.9),
       dict(temperature=0.8, topK=100, topP=0.9, presencePenalty=0.4, frequencyPenalty=0.2),
       dict(temperature=0.0, repetitionPenalty=1.3)]


def _inputs(rows, vocab, seed, configs, coarse=False):
    wl = workloads.make("headline", seed, rows=rows, vocab=vocab)
    logits = np.round(wl.logits) if coarse else wl.logits   # coarse: ties everywhere
    return logits, wl.hist_ids, wl.hist_off, wl.uniforms, configs


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


# large-k rows on coarse logits: the draw lands in a group of equal values,
# ordered by the slot replay (slots in LDS at k = 5000, in the scratch's
# device-memory region at k = 20000)
TIES = [dict(temperature=1.0, topK=20000, topP=0.95),
        dict(temperature=0.8, topK=5000, topP=0.9),
        dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1)]


def test_noalloc_matches_the_allocating_entry_point(sampler):
    calls = [(300, 151936, 1, [MIX[r % len(MIX)] for r in range(300)], False),
             (3, 151936, 2, [MIX[0]] * 3, False),          # split rows: 9 parts each
             (3, 151936, 2, [MIX[0]] * 3, False),          # same configs: no upload
             (40, 50000, 3, [MIX[(r * 7) % len(MIX)] for r in range(40)], False),
             (6, 151936, 4, [TIES[r % len(TIES)] for r in range(6)], True),
             (3, 60000, 5, [TIES[r % len(TIES)] for r in range(3)], True)]
    for rows, vocab, seed, configs, coarse in calls:
        print(f"[gpu] noalloc rows={rows} vocab={vocab} seed={seed} coarse={coarse}", flush=True)
        logits, ids, off, u, cfg = _inputs(rows, vocab, seed, configs, coarse)
        want_t, want_l = _run(sampler, False, logits, ids, off, u, cfg)
        got_t, got_l = _run(sampler, True, logits, ids, off, u, cfg)
        assert np.array_equal(got_t, want_t), (rows, vocab)
        assert np.array_equal(got_l.view(np.uint32), want_l.view(np.uint32)), (rows, vocab)
        ref = logits.copy()
        orc = pyoracle.sample_batch(ref, vocab, ids, off, cfg, u)
        assert np.array_equal(got_l.view(np.uint32), ref.view(np.uint32)), (rows, vocab)
        ok = (got_t == orc.token) | (orc.draw_margin < 1e-6)
        assert ok.all(), (rows, vocab, got_t[~ok], orc.token[~ok])


def test_noalloc_refuses_graph_capture(sampler):
    """Under stream capture the call returns HS_ERR_UNSUPPORTED and enqueues
    nothing (the captured graph is empty); the same stream samples normally
    once the capture has ended."""
    R = hip.runtime()
    vp = ctypes.c_void_p
    R.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    R.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    R.hipGraphGetNodes.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_size_t)]
    R.hipGraphDestroy.argtypes = [vp]
    logits, ids, off, u, cfg = _inputs(4, 50000, 6, [MIX[0]] * 4)
    want_t, _ = _run(sampler, False, logits, ids, off, u, cfg)
    d_l = hip.DeviceArray.from_numpy(logits)
    d_i = hip.DeviceArray.from_numpy(ids)
    d_o = hip.DeviceArray.from_numpy(off)
    d_u = hip.DeviceArray.from_numpy(u)
    d_t = hip.DeviceArray(4, np.int32)
    cfgs = make_configs(cfg, 4)
    st = hip.Stream()
    print("[gpu] noalloc under capture", flush=True)
    hip.check(R.hipStreamBeginCapture(st.handle, 2), "hipStreamBeginCapture")   # relaxed mode
    try:
        with pytest.raises(SamplerError) as e:
            sampler.sample_device_noalloc(d_l.addr, 4, 50000, 50000, d_i.addr, d_o.addr, cfgs,
                                          d_u.addr, d_t.addr, stream=st)
    finally:
        graph = vp()
        hip.check(R.hipStreamEndCapture(st.handle, ctypes.byref(graph)), "hipStreamEndCapture")
    assert e.value.status == 4 and "captured" in str(e.value)
    n = ctypes.c_size_t(0)
    hip.check(R.hipGraphGetNodes(graph, None, ctypes.byref(n)), "hipGraphGetNodes")
    R.hipGraphDestroy(graph)
    assert n.value == 0
    sampler.sample_device_noalloc(d_l.addr, 4, 50000, 50000, d_i.addr, d_o.addr, cfgs, d_u.addr,
                                  d_t.addr, stream=st)
    st.synchronize()
    assert np.array_equal(d_t.download(), want_t)
    st.destroy()


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
