"""GPU parity of the engine's greedy route (src/engine.ts:1600-1601): the
WGSL argmax of src/kernels.ts:1613-1654 through hs_argmax / hs_argmax_device,
against the oracle's step-by-step simulation, on the hand-checked tie cases,
heavy-tie rows, ragged and strided rows, unaligned rows and the full-size
batches.  Every id must be equal."""
import numpy as np
import pytest

from hachiue_amd import hip
from oracle import pyoracle
from tests.test_oracle_wgsl_argmax import KATS

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "whole", "split4"])
def ctx(request, sampler, sampler_whole, sampler_split):
    return {"auto": sampler, "whole": sampler_whole, "split4": sampler_split}[request.param]


def _device(ctx, x, vocab, stride=None, offset=0):
    """hs_argmax_device over rows of x (rows x stride floats), the first row
    `offset` floats past the allocation's start."""
    rows = x.shape[0]
    stride = x.shape[1] if stride is None else stride
    print(f"[gpu] argmax rows={rows} vocab={vocab} stride={stride} offset={offset}", flush=True)
    flat = np.concatenate([np.zeros(offset, np.float32), x.reshape(-1)])
    d = hip.DeviceArray.from_numpy(flat)
    d_tok = hip.DeviceArray(rows, np.int32)
    ctx.argmax_device(d.addr + 4 * offset, rows, stride, vocab, d_tok.addr)
    hip.synchronize()
    return d_tok.download()


def test_known_answers(ctx):
    for name, row, want in KATS:
        got = ctx.argmax(np.ascontiguousarray(row, np.float32))
        assert got.tolist() == [want], name


def test_known_answers_in_one_batch(ctx):
    n = max(r.size for _, r, _ in KATS)
    x = np.full((len(KATS), n), np.nan, np.float32)
    for i, (_, row, _) in enumerate(KATS):
        x[i, :row.size] = row
    # rows shorter than n are padded with NaN, which never wins
    got = _device(ctx, x, n)
    assert got.tolist() == [w for _, _, w in KATS]
    assert got.tolist() == pyoracle.wgsl_argmax(x, n).tolist()


@pytest.mark.parametrize("vocab", [1, 2, 3, 5, 255, 256, 257, 4099, 16385, 65537, 151936])
def test_heavy_ties(ctx, vocab):
    r = np.random.default_rng(vocab)
    x = r.integers(-4, 2, (6, vocab)).astype(np.float32)   # the maximum repeats
    x[1] = np.float32(1.0)                                   # every id ties
    x[2, r.integers(0, vocab, max(1, vocab // 3))] = np.nan
    x[3] = -np.inf
    want = pyoracle.wgsl_argmax(x, vocab)
    assert ctx.argmax(x).tolist() == want.tolist()
    assert _device(ctx, x, vocab).tolist() == want.tolist()


@pytest.mark.parametrize("vocab,stride,offset", [(151669, 151672, 0), (32003, 32005, 0),
                                                 (50257, 50260, 1), (4097, 4097, 3),
                                                 (151936, 151936, 2)])
def test_ragged_strided_unaligned(ctx, vocab, stride, offset):
    r = np.random.default_rng(stride + offset)
    x = r.integers(-3, 3, (5, stride)).astype(np.float32)
    x[:, vocab:] = np.float32(100.0)          # past vocab: never read
    x[4, vocab - 1] = np.float32(50.0)        # the last id wins
    want = pyoracle.wgsl_argmax(x, vocab, stride=stride)
    assert want[4] == vocab - 1
    assert _device(ctx, x, vocab, stride, offset).tolist() == want.tolist()


@pytest.mark.parametrize("rows,vocab", [(1, 151936), (64, 151936), (256, 151936), (16, 262144)])
def test_full_size_batches(sampler, rows, vocab):
    r = np.random.default_rng(rows)
    x = (r.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    x[::2, r.integers(0, vocab, 8)] = np.float32(12.0)   # exact equal spikes on even rows
    want = pyoracle.wgsl_argmax(x, vocab)
    assert _device(sampler, x, vocab).tolist() == want.tolist()


def test_timing_slot(sampler):
    x = np.random.default_rng(0).standard_normal((8, 40000)).astype(np.float32)
    sampler.set_timing(True)
    try:
        sampler.kernel_times()
        _device(sampler, x, 40000)
        ms, calls = sampler.kernel_times()
    finally:
        sampler.set_timing(False)
    assert calls == 1 and ms["argmax_kernel"] > 0
    assert all(v == 0 for k, v in ms.items() if k != "argmax_kernel")


@pytest.mark.parametrize("path", ["sample", "argmax"])
def test_first_call_on_fresh_split_context(path):
    """The first call on a new context grows and clears the split rows'
    arrival counters; that clear must be ordered before the call's kernels on
    the context's own (non-blocking) stream, or a row can count into stale
    memory and never complete (its token stays 0).  Several fresh contexts,
    each used once, on a row whose answer is not 0."""
    from tests.conftest import _context
    x = np.full((1, 151936), -1.0, np.float32)
    x[0, 123457] = 5.0
    for i in range(6):
        s = _context({"HS_ROW_SPLIT": "4"})
        try:
            print(f"[gpu] fresh split context {i}: {path}", flush=True)
            if path == "argmax":
                got = s.argmax(x.copy())
            else:
                got = s.sample_logits_batch(x.copy(), x.shape[1], None, [dict(temperature=0.0)],
                                            np.zeros(1))
            assert got.tolist() == [123457]
        finally:
            s.close()
