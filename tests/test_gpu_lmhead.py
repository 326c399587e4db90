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


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_kquant_heavy_tailed_activations(sampler, fmt):
    """The Q4_K and Q6_K kernels hold x as four int8 limbs per 16-position
    group, exact to 2^-28 of the group's largest |x|.  Hidden states with
    outlier channels (a few positions 100-1000x the rest) and exact zeros
    stay within the bound."""
    wtype, K, N = FORMATS[fmt], 2048, 4099
    rng = np.random.default_rng(77)
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[0, rng.integers(0, K, 12)] *= 1000.0
    x[1, ::5] = 0.0
    x[2] = (rng.standard_normal(K) * np.exp2(rng.integers(-30, 30, K))).astype(np.float32)
    y = run_gemv(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)


# ---- planar Q1_0 / PQ2_0 / PTQ1_0 and Hadamard-folded weights (hs_gemv_device_ex)

from hachiue_amd import sampler as hsamp   # noqa: E402

PLANAR = {"q1_0": o.W_Q1_0, "pq2_0": o.W_PQ2_0, "ptq1_0": o.W_PTQ1_0}


def run_gemv_ex(sampler, wtype, x, w, N, hadamard=False, signs=None, ldx=None, ldy=None):
    """w: the GGUF blocks (raw rows); planar types are split on the host."""
    M, K = x.shape
    ldx = ldx or K
    ldy = ldy or N
    print(f"[gpu] gemv_ex type={wtype} M={M} K={K} N={N} hadamard={hadamard}", flush=True)
    xp = np.zeros((M, ldx), np.float32)
    xp[:, :K] = x
    d_x = hip.DeviceArray.from_numpy(xp)
    keep = [d_x]
    if wtype in PLANAR.values():
        q, sc = hsamp.split_blocks(wtype, w)
        d_w = hip.DeviceArray.from_numpy(q)
        d_s = hip.DeviceArray.from_numpy(sc)
        keep += [d_w, d_s]
        s_addr = d_s.addr
    else:
        d_w = hip.DeviceArray.from_numpy(np.ascontiguousarray(w).reshape(-1))
        keep.append(d_w)
        s_addr = None
    d_sg = None
    if signs is not None:
        d_sg = hip.DeviceArray.from_numpy(np.ascontiguousarray(signs, np.float32))
        keep.append(d_sg)
    wt = hsamp.weights(wtype, N, K, d_w.addr, s_addr, hadamard, d_sg.addr if d_sg else None)
    d_y = hip.DeviceArray.from_numpy(np.full((M, ldy), np.float32(-7.0), np.float32))
    sampler.gemv_device_ex(d_x.addr, M, ldx, wt, d_y.addr, ldy)
    hip.synchronize()
    y = d_y.download()
    assert np.all(y[:, N:] == np.float32(-7.0)), "wrote past N"
    return y[:, :N]


@pytest.mark.parametrize("fmt", list(PLANAR))
@pytest.mark.parametrize("K", [128, 256, 384, 1024, 2048, 4096])
def test_gemv_planar_formats(sampler, fmt, K):
    wtype = PLANAR[fmt]
    rng = np.random.default_rng(K * 7 + wtype)
    N = 1003
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((2, K)).astype(np.float32)
    y = run_gemv_ex(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)


@pytest.mark.parametrize("fmt", list(PLANAR))
def test_gemv_planar_strided_tiny_and_heavy_tailed(sampler, fmt):
    wtype = PLANAR[fmt]
    K = 512
    rng = np.random.default_rng(wtype + 300)
    for N in (1, 2, 5, 17, 33):
        w = random_blocks(wtype, N, K, rng)
        x = rng.standard_normal((3, K)).astype(np.float32)
        # outlier channels, exact zeros and a 2^+-20 range inside a block
        x[1, ::37] *= 300.0
        x[2, :64] = 0.0
        x[2, 64:128] *= np.float32(2.0 ** -20)
        y = run_gemv_ex(sampler, wtype, x, w, N, ldx=K + 5, ldy=N + 3)
        check(wtype, x, w, N, y)


@pytest.mark.parametrize("fmt", list(PLANAR))
def test_gemv_planar_golden_blocks(sampler, fmt):
    """Rows made of the reference's own golden blocks (test/gguf.test.ts:32-115)."""
    import json
    import os
    wtype = PLANAR[fmt]
    path = os.path.join(os.path.dirname(__file__), "golden", "ternary_blocks.json")
    case = [c for c in json.load(open(path))["cases"] if c["type"] == wtype][0]
    blk = np.array(case["block"], np.uint8)
    K, N = 1024, 40
    w = np.tile(blk, (N, K // 128))
    x = np.random.default_rng(3).standard_normal((2, K)).astype(np.float32)
    y = run_gemv_ex(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)
    row = np.tile(np.array(case["weights"], np.float64), K // 128)
    want = (x.astype(np.float64) @ row)[:, None]
    bound = TOL * (np.abs(x.astype(np.float64)) @ np.abs(row))[:, None]
    assert np.all(np.abs(y - want) <= bound)


@pytest.mark.parametrize("fmt,N", [("q1_0", 151669), ("pq2_0", 151936), ("ptq1_0", 151936)])
def test_gemv_planar_full_vocabulary(sampler, fmt, N):
    wtype = PLANAR[fmt]
    K = 2048
    rng = np.random.default_rng(N + wtype)
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = run_gemv_ex(sampler, wtype, x, w, N)
    check(wtype, x, w, N, y)


def test_gemv_planar_nonfinite_input(sampler):
    wtype, K, N = o.W_PQ2_0, 256, 20
    rng = np.random.default_rng(5)
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[1, 200] = np.nan
    x[2, 3] = np.inf
    y = run_gemv_ex(sampler, wtype, x, w, N)
    assert np.all(np.isnan(y[1])) and np.all(np.isnan(y[2]))
    check(wtype, x[:1], w, N, y[:1])


@pytest.mark.parametrize("with_signs", [False, True])
def test_hadamard_rotation_bit_exact(sampler, with_signs):
    """With identity F32 weights the GEMV returns its rotated input exactly:
    it equals the oracle's rotation (src/kernels.ts:177-227) bit for bit."""
    K, M = 1024, 3
    rng = np.random.default_rng(9)
    x = rng.standard_normal((M, K)).astype(np.float32)
    eye = np.eye(K, dtype=np.float32).view(np.uint8)
    signs = np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32) if with_signs else None
    y = run_gemv_ex(sampler, o.W_F32, x, eye, K, hadamard=True, signs=signs, ldx=K + 3)
    want = o.hadamard512(x, signs)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q6_k", "q4_0", "q1_0", "ptq1_0"])
def test_hadamard_folded_weights(sampler, fmt):
    wtype = {**FORMATS, **PLANAR}[fmt]
    K, N = 2048, 777
    rng = np.random.default_rng(wtype + 17)
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((2, K)).astype(np.float32)
    signs = np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32)
    y = run_gemv_ex(sampler, wtype, x, w, N, hadamard=True, signs=signs)
    check(wtype, o.hadamard512(x, signs), w, N, y)


def test_lm_head_then_sample_planar_folded(sampler):
    """A PTQ1_0, Hadamard-folded lm_head and the sampler on one stream."""
    wtype, K, N, M = o.W_PTQ1_0, 1024, 151936, 3
    rng = np.random.default_rng(21)
    w = random_blocks(wtype, N, K, rng, scale=0.05)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hist = [rng.integers(0, N, 64).astype(np.int32) for _ in range(M)]
    off = np.zeros(M + 1, np.int64)
    for r, h in enumerate(hist):
        off[r + 1] = off[r] + h.size
    ids = np.concatenate(hist)
    cfgs = [dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
            dict(temperature=0.0), dict(temperature=1.0, topK=200, topP=0.95)]
    u = rng.random(M)
    q, sc = hsamp.split_blocks(wtype, w)
    d_x = hip.DeviceArray.from_numpy(x)
    d_q = hip.DeviceArray.from_numpy(q)
    d_s = hip.DeviceArray.from_numpy(sc)
    d_l = hip.DeviceArray((M, N), np.float32)
    d_ids = hip.DeviceArray.from_numpy(ids)
    d_off = hip.DeviceArray.from_numpy(off)
    d_u = hip.DeviceArray.from_numpy(u)
    d_t = hip.DeviceArray(M, np.int32)
    wt = hsamp.weights(wtype, N, K, d_q.addr, d_s.addr, True, None)
    print("[gpu] lm_head (ptq1_0, folded) + sample", flush=True)
    sampler.lm_head_sample_device_ex(d_x.addr, M, K, wt, d_l.addr, N, d_ids.addr, d_off.addr,
                                     cfgs, d_u.addr, d_t.addr)
    hip.synchronize()
    tokens, pen = d_t.download(), d_l.download()
    raw = run_gemv_ex(sampler, wtype, x, w, N, hadamard=True)
    check(wtype, o.hadamard512(x), w, N, raw)
    ref = raw.copy()
    res = o.sample_batch(ref, N, ids, off, cfgs, u)
    assert tokens.tolist() == res.token.tolist()
    assert np.array_equal(pen.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_gemv_kquant_nonfinite_input(sampler, fmt):
    """The Q4_K and Q6_K matrix-core kernels hold x as integer limbs: a row of
    x with a NaN or an infinity gives NaN for every result of that row."""
    wtype, K, N = FORMATS[fmt], 512, 40
    rng = np.random.default_rng(6)
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[1, 300] = np.nan
    x[2, 7] = -np.inf
    y = run_gemv(sampler, wtype, x, w, N)
    assert np.all(np.isnan(y[1])) and np.all(np.isnan(y[2]))
    check(wtype, x[:1], w, N, y[:1])
