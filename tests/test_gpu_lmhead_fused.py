"""GPU parity of the lm_head GEMVs that sample their own rows in one
launch (hs_lm_head_sample_device_ex; the planar, Q4_K and Q6_K formats
when every row is greedy or takes k <= 64 candidates with at most the
repetition penalty, the vector-unit formats when every row is greedy;
src/engine.ts:1493-1531 then src/sampler.ts).
The logits it leaves (penalised where the history asks, src/sampler.ts:
24-33) must equal, bit for bit, the GEMV's own output with the oracle's
penalties applied, and every token the oracle's on those logits; the same
call on a context that always takes two launches (HS_LMHEAD_FUSE=0) must
give the same tokens and logits."""
import numpy as np
import pytest

from hachiue_amd import hip
from hachiue_amd import sampler as hsamp
from oracle import pyoracle as o
from tests.conftest import _context
from tests.test_gpu_lmhead import PLANAR, check, run_gemv_ex
from tests.test_oracle_lmhead import random_blocks

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def unfused():
    s = _context({"HS_LMHEAD_FUSE": "0"})
    yield s
    s.close()


@pytest.fixture(scope="module")
def fctx():
    """A context that takes the one launch wherever it applies (sampling
    rows too; by default those take two launches)."""
    s = _context({"HS_LMHEAD_FUSE": "2"})
    yield s
    s.close()


def lm_head_sample(ctx, wtype, x, w, N, hists, cfgs, u, hadamard=False):
    """One hs_lm_head_sample_device_ex call: (tokens, logits left behind)."""
    M, K = x.shape
    if wtype in PLANAR.values():
        q, sc = hsamp.split_blocks(wtype, w)
    else:   # GGUF blocks as they are
        q, sc = np.ascontiguousarray(w, np.uint8).reshape(-1), None
    off = np.zeros(M + 1, np.int64)
    for r, h in enumerate(hists):
        off[r + 1] = off[r] + len(h)
    ids = np.concatenate([np.asarray(h, np.int32) for h in hists]) if off[-1] else \
        np.zeros(1, np.int32)
    d_x = hip.DeviceArray.from_numpy(x)
    d_q = hip.DeviceArray.from_numpy(q)
    d_s = hip.DeviceArray.from_numpy(sc) if sc is not None else None
    d_l = hip.DeviceArray.from_numpy(np.full((M, N), np.float32(-7.0), np.float32))
    d_ids = hip.DeviceArray.from_numpy(ids)
    d_off = hip.DeviceArray.from_numpy(off)
    d_u = hip.DeviceArray.from_numpy(np.asarray(u, np.float64))
    d_t = hip.DeviceArray.from_numpy(np.full(M, -5, np.int32))
    wt = hsamp.weights(wtype, N, K, d_q.addr, d_s.addr if d_s else None, hadamard, None)
    print(f"[gpu] fused lm_head+sample type={wtype} M={M} K={K} N={N} cfgs={cfgs}", flush=True)
    ctx.lm_head_sample_device_ex(d_x.addr, M, K, wt, d_l.addr, N, d_ids.addr, d_off.addr, cfgs,
                                 d_u.addr, d_t.addr)
    hip.synchronize()
    return d_t.download(), d_l.download(), ids, off


def expect(sampler, wtype, x, w, N, ids, off, cfgs, u, hadamard=False):
    raw = run_gemv_ex(sampler, wtype, x, w, N, hadamard=hadamard)
    ref = raw.copy()
    res = o.sample_batch(ref, N, ids, off, cfgs, np.asarray(u, np.float64))
    return raw, ref, res


CFGS = [dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
        dict(temperature=0.0),
        dict(temperature=0.0, repetitionPenalty=1.3),
        dict(),                                                   # 0.6, 20, 0.95
        dict(temperature=1.0, topK=64, topP=1.0, minP=0.02, repetitionPenalty=0.8),
        dict(temperature=0.9, topK=1)]


FUSED = dict(PLANAR, q4_k=o.W_Q4_K, q6_k=o.W_Q6_K)


@pytest.mark.parametrize("fmt", list(FUSED))
def test_fused_full_vocabulary(sampler, fctx, unfused, fmt):
    wtype, K, N = FUSED[fmt], 1024, 151936
    rng = np.random.default_rng(31 + wtype)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    M = len(CFGS)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hists = [rng.integers(0, N, 200) for _ in range(M)]
    hists[2] = np.concatenate([hists[2], [0, N - 1, 0, -3, N + 5]])   # edges and outside ids
    u = rng.random(M)
    tok, pen, ids, off = lm_head_sample(fctx, wtype, x, w, N, hists, CFGS, u)
    raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, CFGS, u)
    check(wtype, x, w, N, raw)
    assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
    ok = (tok == res.token) | (res.draw_margin < 1e-6)
    assert ok.all(), (tok.tolist(), res.token.tolist())
    tok2, pen2, _, _ = lm_head_sample(unfused, wtype, x, w, N, hists, CFGS, u)
    assert tok.tolist() == tok2.tolist()
    assert np.array_equal(pen.view(np.uint32), pen2.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q1_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("N", [1, 15, 17, 1000, 4099, 65537])
def test_fused_small_and_ragged_vocabularies(sampler, fctx, N, fmt):
    wtype, K = FUSED[fmt], 256
    rng = np.random.default_rng(N)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    cfgs = [dict(temperature=0.8, topK=40, topP=0.95, repetitionPenalty=1.2),
            dict(temperature=0.0, repetitionPenalty=1.2), dict(temperature=1.3, topK=64)]
    M = len(cfgs)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hists = [rng.integers(0, N, 50) for _ in range(M)]
    u = rng.random(M)
    tok, pen, ids, off = lm_head_sample(fctx, wtype, x, w, N, hists, cfgs, u)
    raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, cfgs, u)
    assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
    ok = (tok == res.token) | (res.draw_margin < 1e-6)
    assert ok.all(), (tok.tolist(), res.token.tolist())


@pytest.mark.parametrize("fmt", list(FUSED))
def test_fused_equal_logits_replay(sampler, fctx, fmt):
    """Every row of W equal: all logits of a row are equal, so the top-k order
    is the slot history of src/sampler.ts:55-69 (here the first k ids) and
    the draw falls in a group of equal values: the last workgroup replays."""
    wtype, K, N = FUSED[fmt], 512, 40000
    rng = np.random.default_rng(7)
    one = random_blocks(wtype, 1, K, rng, scale=0.05)
    w = np.repeat(one, N, axis=0)
    cfgs = [dict(temperature=0.7, topK=40, topP=0.9), dict(temperature=1.0, topK=64, topP=1.0),
            dict(temperature=0.0), dict(temperature=0.8, topK=5, repetitionPenalty=1.5)]
    M = len(cfgs)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hists = [[], [], [], [3, 0, 39999, 17]]
    u = rng.random(M)
    tok, pen, ids, off = lm_head_sample(fctx, wtype, x, w, N, hists, cfgs, u)
    raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, cfgs, u)
    assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
    assert tok.tolist() == res.token.tolist()


def test_fused_hadamard_folded_and_mixed_rows(sampler, fctx, unfused):
    """A folded PQ2_0 lm_head (the rotation runs first); then a batch with a
    k > 64 row, which takes the two launches, gives the same results."""
    wtype, K, N = o.W_PQ2_0, 1024, 151669
    rng = np.random.default_rng(3)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    x = rng.standard_normal((3, K)).astype(np.float32)
    hists = [rng.integers(0, N, 64) for _ in range(3)]
    u = rng.random(3)
    for cfgs in ([dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
                  dict(temperature=0.0), dict(topK=10)],
                 [dict(temperature=0.7, topK=40), dict(temperature=1.0, topK=300, topP=0.95),
                  dict(temperature=0.0)]):
        tok, pen, ids, off = lm_head_sample(fctx, wtype, x, w, N, hists, cfgs, u, hadamard=True)
        raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, cfgs, u, hadamard=True)
        assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
        ok = (tok == res.token) | (res.draw_margin < 1e-6)
        assert ok.all(), (tok.tolist(), res.token.tolist())
        tok2, pen2, _, _ = lm_head_sample(unfused, wtype, x, w, N, hists, cfgs, u, hadamard=True)
        assert tok.tolist() == tok2.tolist()
        assert np.array_equal(pen.view(np.uint32), pen2.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q1_0", "q4_k", "q6_k"])
def test_fused_repeated_calls_reset_state(sampler, fctx, fmt):
    """Per-row state (pool, bound, counters) is zero between calls: the same
    call three times, then a call with fewer rows, each exact."""
    wtype, K, N = FUSED[fmt], 512, 151936
    rng = np.random.default_rng(44)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    x = rng.standard_normal((4, K)).astype(np.float32)
    cfgs = [dict(temperature=0.7, topK=40, topP=0.9), dict(temperature=0.0),
            dict(temperature=1.1, topK=64), dict(topK=3)]
    hists = [rng.integers(0, N, 10) for _ in range(4)]
    u = rng.random(4)
    want = None
    for rep in range(3):
        tok, pen, ids, off = lm_head_sample(fctx, wtype, x, w, N, hists, cfgs, u)
        if want is None:
            raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, cfgs, u)
            assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
            want = res.token.tolist()
        assert tok.tolist() == want
    tok, pen, ids, off = lm_head_sample(fctx, wtype, x[:2], w, N, hists[:2], cfgs[:2], u[:2])
    assert tok.tolist() == want[:2]


@pytest.mark.parametrize("fmt", ["q1_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("cfg", [dict(topK=40), dict(temperature=0.0, repetitionPenalty=1.2)])
def test_fused_is_one_launch(sampler, fctx, unfused, fmt, cfg):
    """The qualifying call launches the lm_head kernel alone (the sampler's
    kernels do not run); the two-launch context also runs the sampler's
    kernel.  By default a call with a sampling row takes two launches.
    Every call gives the oracle's token."""
    wtype, K, N = FUSED[fmt], 256, 20000
    rng = np.random.default_rng(2)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    x = rng.standard_normal((1, K)).astype(np.float32)
    default_fused = cfg.get("temperature", 0.6) <= 0
    for ctx, fused in ((fctx, True), (sampler, default_fused), (unfused, False)):
        ctx.set_timing(True)
        ctx.kernel_times()
        tok, pen, ids, off = lm_head_sample(ctx, wtype, x, w, N, [[1, 2]], [cfg], [0.5])
        raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, [cfg], [0.5])
        assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
        assert (tok[0] == res.token[0]) or res.draw_margin[0] < 1e-6
        ms, calls = ctx.kernel_times()
        ctx.set_timing(False)
        others = {k: v for k, v in ms.items() if v > 0 and k != "gemv_kernel"}
        assert ms["gemv_kernel"] > 0
        assert (others == {}) == fused, others


BLOCK = {"f32": o.W_F32, "q4_0": o.W_Q4_0, "q4_1": o.W_Q4_1}


@pytest.mark.parametrize("fmt", list(BLOCK))
@pytest.mark.parametrize("K", [1024, 4096])
def test_fused_greedy_vector_formats(sampler, fctx, unfused, fmt, K):
    """Every row greedy on the vector-unit formats (both lane layouts: a row
    on `seg` lanes at K 1024, on all 64 with two units each at K 4096): one
    launch when HS_LMHEAD_FUSE=2 asks for it (by default two: the one launch
    is slower on these formats), the tokens the oracle's on the GEMV's own
    logits (first index of the maximum, logit 0 NaN -> 0), the penalised
    logits bit for bit, and the same results as two launches.  Rows with a
    sampling row take two launches."""
    wtype = BLOCK[fmt]
    N = 40000 if fmt == "f32" else 151936
    rng = np.random.default_rng(K + wtype)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    cfgs = [dict(temperature=0.0), dict(temperature=0.0, repetitionPenalty=1.3),
            dict(temperature=-1.0, repetitionPenalty=0.7)]
    M = len(cfgs)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hists = [rng.integers(0, N, 100) for _ in range(M)]
    u = rng.random(M)
    for ctx, fused in ((fctx, True), (sampler, False), (unfused, False)):
        ctx.set_timing(True)
        ctx.kernel_times()
        tok, pen, ids, off = lm_head_sample(ctx, wtype, x, w, N, hists, cfgs, u)
        ms, calls = ctx.kernel_times()
        ctx.set_timing(False)
        others = {k: v for k, v in ms.items() if v > 0 and k != "gemv_kernel"}
        assert (others == {}) == fused, others
        raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, cfgs, u)
        assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
        assert tok.tolist() == res.token.tolist()
    mixed = cfgs[:2] + [dict(temperature=0.7, topK=40)]
    tok, pen, ids, off = lm_head_sample(fctx, wtype, x, w, N, hists, mixed, u)
    raw, ref, res = expect(sampler, wtype, x, w, N, ids, off, mixed, u)
    assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))
    assert ((tok == res.token) | (res.draw_margin < 1e-6)).all()
