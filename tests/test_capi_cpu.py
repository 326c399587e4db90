"""The C-ABI library on a machine without a GPU: it loads, exports every
entry point include/hachiue_sampler.h declares, and reports errors through
status codes and hs_last_error() instead of crashing.  No compute call is
made here."""
import ctypes
import os
import re

import pytest

from hachiue_amd import sampler

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hachiue_sampler.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hs_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(sampler.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(sampler.EXPORTS)


def test_abi_version_and_defaults():
    L = sampler.lib()
    assert L.hs_abi_version() == 1
    c = sampler.SampleConfigC()
    L.hs_config_default(ctypes.byref(c))
    # src/sampler.ts:18-22
    assert (c.temperature, c.top_k, c.top_p, c.min_p, c.repetition_penalty) == (0.6, 20, 0.95, 0, 1)
    assert (c.presence_penalty, c.frequency_penalty) == (0, 0)
    assert ctypes.sizeof(sampler.SampleConfigC) == 56


def test_null_context_is_an_argument_error():
    L = sampler.lib()
    tok = ctypes.c_int32(-7)
    cfg = sampler.resolve_config({})
    logits = (ctypes.c_float * 4)(1, 2, 3, 4)
    rc = L.hs_sample_logits(None, logits, 4, None, 0, ctypes.byref(cfg), 0.5, ctypes.byref(tok))
    assert rc == 1
    assert b"null context" in L.hs_last_error()
    assert L.hs_context_destroy(None) == 0


def test_context_without_device_fails_cleanly():
    from hachiue_amd import hip
    if hip.device_count() > 0:
        pytest.skip("a GPU is visible")
    L = sampler.lib()
    ctx = ctypes.c_void_p()
    rc = L.hs_context_create(0, ctypes.byref(ctx))
    assert rc == 2   # HS_ERR_HIP
    assert ctx.value is None
    assert b"no HIP device" in L.hs_last_error()
    with pytest.raises(sampler.SamplerError) as e:
        sampler.Sampler(0)
    assert e.value.status == 2


def test_timing_calls_reject_null_context():
    L = sampler.lib()
    assert L.hs_context_set_timing(None, 1) == 1
    ms = (ctypes.c_double * 4)()
    assert L.hs_context_kernel_times(None, ms, 4, None) == 1


def test_split_blocks_matches_the_block_layouts():
    """hs_split_blocks (host) puts each block's quant bytes and binary16
    scale where the planar GEMV reads them (src/engine.ts:80-175)."""
    import numpy as np
    rng = np.random.default_rng(1)
    for wtype, qb, scale_at in ((41, 16, 0), (142, 32, 0), (143, 26, 26)):
        blocks = rng.integers(0, 256, (7, qb + 2), dtype=np.uint8)
        q, sc = sampler.split_blocks(wtype, blocks)
        for b in range(7):
            want_q = np.concatenate([blocks[b, :scale_at], blocks[b, scale_at + 2:]])
            assert np.array_equal(q[b * qb:(b + 1) * qb], want_q)
            assert np.array_equal(sc[2 * b:2 * b + 2], blocks[b, scale_at:scale_at + 2])
    with pytest.raises(sampler.SamplerError) as e:
        sampler._check(sampler.lib().hs_split_blocks(14, None, 1, None, None))
    assert e.value.status == 1


def test_gemv_ex_rejects_bad_weights_without_a_gpu():
    L = sampler.lib()
    w = sampler.weights(41, 10, 256, None)
    rc = L.hs_gemv_device_ex(None, None, 1, 256, ctypes.byref(w), None, 10, None)
    assert rc == 1 and b"null context" in L.hs_last_error()
