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
