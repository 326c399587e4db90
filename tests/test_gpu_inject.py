"""Error paths under injected HIP failures (HS_INJECT_HIP_FAILURE, read at
context creation: the n-th checked HIP runtime call after it reports
hipErrorOutOfMemory without being made).  For every n that the call path
reaches, the entry point returns HS_ERR_HIP with the failing call named,
leaves the caller's logits untouched, and the same context then samples
correctly (tokens and penalised logits equal to the oracle's).  The failure
is made on the host: no kernel faults."""
import numpy as np
import pytest

from hachiue_amd import hip, workloads
from hachiue_amd.sampler import SamplerError
from oracle import pyoracle
from tests.conftest import _context

pytestmark = pytest.mark.gpu


def _reset():
    """A context created with injection off resets the process-wide counter."""
    _context({"HS_INJECT_HIP_FAILURE": "-1"}).close()


def _want(wl):
    ref = wl.logits.copy()
    res = pyoracle.sample_batch(ref, wl.vocab, wl.hist_ids, wl.hist_off, wl.configs, wl.uniforms)
    return res.token, ref


def test_host_entry_point_recovers_after_each_injected_failure():
    _reset()   # the once-per-device set-up is done before any injection
    wl = workloads.make("perrow256", 4, rows=6, vocab=30000)   # presence/frequency: pre-pass too
    want_tok, want_logits = _want(wl)
    failures = 0
    for n in range(64):
        print(f"[gpu] inject at HIP call {n} (host batch)", flush=True)
        s = _context({"HS_INJECT_HIP_FAILURE": str(n)})
        try:
            logits = wl.logits.copy()
            try:
                s.sample_logits_batch(logits, wl.vocab, (wl.hist_ids, wl.hist_off), wl.configs,
                                      wl.uniforms)
                injected = False
            except SamplerError as e:
                injected = True
                assert e.status == 2 and "out of memory" in str(e), str(e)
                assert np.array_equal(logits.view(np.uint32), wl.logits.view(np.uint32))
            _reset()
            logits = wl.logits.copy()
            tok = s.sample_logits_batch(logits, wl.vocab, (wl.hist_ids, wl.hist_off), wl.configs,
                                        wl.uniforms)
            assert tok.tolist() == want_tok.tolist()
            assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
        finally:
            s.close()
            _reset()
        if not injected:
            break
        failures += 1
    assert failures >= 4, failures


def test_device_entry_point_recovers_after_each_injected_failure():
    _reset()
    wl = workloads.make("batch64", 5, rows=8, vocab=40000)
    want_tok, want_logits = _want(wl)
    failures = 0
    for n in range(64):
        print(f"[gpu] inject at HIP call {n} (device batch)", flush=True)
        s = _context({"HS_INJECT_HIP_FAILURE": str(n)})
        try:
            d_l = hip.DeviceArray.from_numpy(wl.logits)
            d_i = hip.DeviceArray.from_numpy(wl.hist_ids)
            d_o = hip.DeviceArray.from_numpy(wl.hist_off)
            d_u = hip.DeviceArray.from_numpy(wl.uniforms)
            d_t = hip.DeviceArray(wl.rows, np.int32)
            try:
                s.sample_device(d_l.addr, wl.rows, wl.vocab, wl.vocab, d_i.addr, d_o.addr,
                                wl.configs, d_u.addr, d_t.addr)
                hip.synchronize()
                injected = False
            except SamplerError as e:
                injected = True
                assert e.status == 2 and "out of memory" in str(e), str(e)
            hip.synchronize()
            _reset()
            d_l = hip.DeviceArray.from_numpy(wl.logits)
            s.sample_device(d_l.addr, wl.rows, wl.vocab, wl.vocab, d_i.addr, d_o.addr, wl.configs,
                            d_u.addr, d_t.addr)
            hip.synchronize()
            assert d_t.download().tolist() == want_tok.tolist()
            assert np.array_equal(d_l.download().view(np.uint32), want_logits.view(np.uint32))
        finally:
            s.close()
            _reset()
        if not injected:
            break
        failures += 1
    assert failures >= 2, failures


def test_noalloc_entry_point_recovers_after_each_injected_failure():
    """Two contexts share the GPU's scratch array.  Context B uploads its
    plans; context A's call with other configs fails at its n-th HIP call
    (the capture check, the plan copy, the list copy or the event record).
    Whatever A's upload left in the scratch, B's next call with its old
    configs must upload them again (no stale "same" path), and both contexts
    then sample exactly (tokens and penalised logits equal to the oracle's)."""
    _reset()
    wa = workloads.make("batch64", 6, rows=8, vocab=40000)
    wb = workloads.make("perrow256", 7, rows=5, vocab=40000)
    want_a, want_la = _want(wa)
    want_b, want_lb = _want(wb)

    def run(s, wl):
        d_l = hip.DeviceArray.from_numpy(wl.logits)
        d_i = hip.DeviceArray.from_numpy(wl.hist_ids)
        d_o = hip.DeviceArray.from_numpy(wl.hist_off)
        d_u = hip.DeviceArray.from_numpy(wl.uniforms)
        d_t = hip.DeviceArray(wl.rows, np.int32)
        s.sample_device_noalloc(d_l.addr, wl.rows, wl.vocab, wl.vocab, d_i.addr, d_o.addr,
                                wl.configs, d_u.addr, d_t.addr)
        hip.synchronize()
        return d_t.download(), d_l.download()

    failures = 0
    b = _context({})
    try:
        for n in range(16):
            print(f"[gpu] inject at HIP call {n} (no-allocation, two contexts)", flush=True)
            tok, lg = run(b, wb)
            assert tok.tolist() == want_b.tolist()
            a = _context({"HS_INJECT_HIP_FAILURE": str(n)})
            try:
                try:
                    run(a, wa)
                    injected = False
                except SamplerError as e:
                    injected = True
                    assert e.status == 2 and "out of memory" in str(e), str(e)
                hip.synchronize()
                _reset()
                tok, lg = run(b, wb)
                assert tok.tolist() == want_b.tolist()
                assert np.array_equal(lg.view(np.uint32), want_lb.view(np.uint32))
                tok, lg = run(a, wa)
                assert tok.tolist() == want_a.tolist()
                assert np.array_equal(lg.view(np.uint32), want_la.view(np.uint32))
            finally:
                a.close()
                _reset()
            if not injected:
                break
            failures += 1
    finally:
        b.close()
    assert failures >= 3, failures
