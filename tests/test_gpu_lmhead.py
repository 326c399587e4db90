"""GPU parity of the lm_head GEMV (hs_gemv_device, src/engine.ts:1493-1515)
and of the lm_head + sampler call (hs_lm_head_sample_device) against the
oracle: every output within the binary32 rounding bound of the exact
binary64 product (|y - exact| <= 2^-16 * sum_k |x_k w_k|, the bound the
reference's own order meets in tests/test_oracle_lmhead.py), on every
format, lane layout (K from 256 to 4096), ragged N, strided x and y, and the
full-size vocabulary."""
import numpy as np
import pytest

from hachiue_amd import hip
from oracle import pyoracle as o
from tests.test_oracle_lmhead import random_blocks

pytestmark = pytest.mark.gpu

TOL = 2.0 ** -16
FORMATS = {"f32": o.W_F32, "q4_0": o.W_Q4_0, "q4_1": o.W_Q4_1, "q4_k": o.W_Q4_K,
           "q6_k": o.W_Q6_K}


def run_gemv(sampler, wtype, x, w, N, ldx=None, ldy=None):
    M, K = x.shape
    ldx = ldx or K
    ldy = ldy or N
    print(f"[gpu] gemv type={wtype} M={M} K={K} N={N} ldx={ldx} ldy={ldy}", flush=True)
    xp = np.zeros((M, ldx), np.float32)
    xp[:, :K] = x
    d_x = hip.DeviceArray.from_numpy(xp)
    d_w = hip.DeviceArray.from_numpy(np.ascontiguousarray(w).reshape(-1))
    d_y = hip.DeviceArray.from_numpy(np.full((M, ldy), np.float32(-7.0), np.float32))
    sampler.gemv_device(d_x.addr, M, ldx, K, d_w.addr, wtype, N, d_y.addr, ldy)
    hip.synchronize()
    y = d_y.download()
    assert np.all(y[:, N:] == np.float32(-7.0)), "wrote past N"
    return y[:, :N]


def check(wtype, x, w, N, y):
    exact, mag = o.gemv_exact(wtype, x, w, N)
    err = np.abs(y.astype(np.float64) - exact)
    assert np.all(err <= TOL * mag + 1e-30), (wtype, float(np.max(err / (mag + 1e-30))))


@pytest.mark.parametrize("fmt", list(FORMATS))
@pytest.mark.parametrize("K", [256, 512, 1024, 1536, 2048, 4096])
def test_gemv_formats_and_lane_layouts(sampler, fmt, K):
    wtype = FORMATS[fmt]
    B, _ = o.block_spec(wtype)
    if K % max(B, 32):
        pytest.skip("K not a multiple of the block")
    rng = np.random.default_rng(K * 31 + wtype)
    N = 1003                       # not a multiple of any rows-per-step
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((2, K)).astype(np.float32)
    y = run_gemv(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)


@pytest.mark.parametrize("fmt", list(FORMATS))
def test_gemv_strided_and_tiny(sampler, fmt):
    wtype = FORMATS[fmt]
    K = 256
    rng = np.random.default_rng(wtype + 100)
    for N in (1, 2, 5, 17):
        w = random_blocks(wtype, N, K, rng)
        x = rng.standard_normal((3, K)).astype(np.float32)
        y = run_gemv(sampler, wtype, x, w, N, ldx=K + 5, ldy=N + 3)
        check(wtype, x, w, N, y)


@pytest.mark.parametrize("fmt,K", [("q6_k", 2048), ("q6_k", 1536), ("q4_k", 4096),
                                   ("q4_0", 1024)])
def test_gemv_full_vocabulary(sampler, fmt, K):
    wtype = FORMATS[fmt]
    rng = np.random.default_rng(K)
    N = 151936
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = run_gemv(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)


def test_lm_head_then_sample(sampler):
    """Logits stay on the GPU between the GEMV and the sampler; the tokens
    equal the oracle's on the same logits, and the penalised logits match."""
    wtype, K, N, M = o.W_Q6_K, 1024, 151936, 4
    rng = np.random.default_rng(11)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hist = [rng.integers(0, N, 64).astype(np.int32) for _ in range(M)]
    off = np.zeros(M + 1, np.int64)
    for r, h in enumerate(hist):
        off[r + 1] = off[r] + h.size
    ids = np.concatenate(hist)
    cfgs = [dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
            dict(temperature=0.0),
            dict(temperature=1.0, topK=200, topP=0.95),
            dict(temperature=0.8, topK=0, topP=1.0, minP=0.05)]
    u = rng.random(M)
    d_x = hip.DeviceArray.from_numpy(x)
    d_w = hip.DeviceArray.from_numpy(w.reshape(-1))
    d_l = hip.DeviceArray((M, N), np.float32)
    d_ids = hip.DeviceArray.from_numpy(ids)
    d_off = hip.DeviceArray.from_numpy(off)
    d_u = hip.DeviceArray.from_numpy(u)
    d_t = hip.DeviceArray(M, np.int32)
    print("[gpu] lm_head + sample", flush=True)
    sampler.lm_head_sample_device(d_x.addr, M, K, K, d_w.addr, wtype, N, d_l.addr, N, d_ids.addr,
                                  d_off.addr, cfgs, d_u.addr, d_t.addr)
    hip.synchronize()
    tokens, pen = d_t.download(), d_l.download()
    # the logits before the penalties: the same GEMV alone
    raw = run_gemv(sampler, wtype, x, w, N)
    check(wtype, x, w, N, raw)
    ref = raw.copy()
    res = o.sample_batch(ref, N, ids, off, cfgs, u)
    assert tokens.tolist() == res.token.tolist()
    assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))


def test_q6k_heavy_tailed_activations(sampler):
    """The Q6_K kernel holds x as four int8 limbs per 16-position scale group,
    exact to 2^-28 of the group's largest |x|.  Hidden states with outlier
    channels (a few positions 100-1000x the rest) and exact zeros stay within
    the bound."""
    wtype, K, N = o.W_Q6_K, 2048, 4099
    rng = np.random.default_rng(77)
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[0, rng.integers(0, K, 12)] *= 1000.0
    x[1, ::5] = 0.0
    x[2] = (rng.standard_normal(K) * np.exp2(rng.integers(-30, 30, K))).astype(np.float32)
    y = run_gemv(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)
