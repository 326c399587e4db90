"""The lm_head GEMV oracle (oracle/lmhead_oracle.c) pinned without the C
code's own formulas:

- the reference's golden Q4_0 / Q4_1 blocks (test/gguf.test.ts:117-143) and
  its Q1_0 / PQ2_0 / PTQ1_0 blocks (test/gguf.test.ts:32-115);
- the 512-wide Hadamard rotation against the dense Sylvester matrix, its
  own inverse, and exact answers on integer inputs (test/gguf.test.ts:146-181);
- binary16 conversion against numpy's float16 on every bit pattern;
- dequantisation against an independent vectorised numpy decoder (PTQ1_0
  trits as base-3 digits of floor(243 b / 256));
- K-quant bit layouts by round trips through packers written from the block
  layouts (scale index = weight / 16 for Q6_K, the 6-bit scale/min packing
  of Q4_K), so that a wrong shift or index in the decoder fails;
- the exact GEMV against numpy's float64 product of the decoded weights;
- the reference-order binary32 GEMV within the rounding bound of its sum.
"""
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as o

TYPES = [o.W_F32, o.W_Q4_0, o.W_Q4_1, o.W_Q4_K, o.W_Q6_K]
TERNARY = [o.W_Q1_0, o.W_PQ2_0, o.W_PTQ1_0]


def f16_bytes(vals):
    return np.asarray(vals, np.float16).view(np.uint8)


def random_blocks(wtype, n_rows, K, rng, scale=0.02):
    """Rows of valid blocks: random quants, finite scales near `scale`."""
    B, BB = o.block_spec(wtype)
    nb = K // B
    if wtype == o.W_F32:
        return (rng.standard_normal((n_rows, K)) * scale).astype(np.float32).view(np.uint8)
    raw = rng.integers(0, 256, (n_rows, nb, BB), dtype=np.uint8)
    d = (rng.random((n_rows, nb)) * 2 * scale).astype(np.float16)
    if wtype in (o.W_Q4_0, o.W_Q4_1, o.W_Q4_K):
        raw[:, :, 0:2] = d.view(np.uint8).reshape(n_rows, nb, 2)
    if wtype == o.W_Q4_1:
        m = (rng.standard_normal((n_rows, nb)) * scale).astype(np.float16)
        raw[:, :, 2:4] = m.view(np.uint8).reshape(n_rows, nb, 2)
    if wtype == o.W_Q4_K:
        dmin = (rng.random((n_rows, nb)) * scale).astype(np.float16)
        raw[:, :, 2:4] = dmin.view(np.uint8).reshape(n_rows, nb, 2)
    if wtype == o.W_Q6_K:
        raw[:, :, 208:210] = d.view(np.uint8).reshape(n_rows, nb, 2)
    if wtype in (o.W_Q1_0, o.W_PQ2_0):
        raw[:, :, 0:2] = d.view(np.uint8).reshape(n_rows, nb, 2)
    if wtype == o.W_PTQ1_0:
        raw[:, :, 26:28] = d.view(np.uint8).reshape(n_rows, nb, 2)
    return raw.reshape(n_rows, nb * BB)


# ---- independent numpy decoder (exact weights as float64) -------------------

def np_weights(wtype, w, K):
    B, BB = o.block_spec(wtype)
    n = w.shape[0]
    if wtype == o.W_F32:
        return w.view(np.float32).astype(np.float64).reshape(n, K)
    b = w.reshape(n, K // B, BB)
    h = lambda a, i: b[:, :, i:i + 2].copy().view(np.float16)[..., 0].astype(np.float64)
    if wtype in (o.W_Q4_0, o.W_Q4_1):
        qs = b[:, :, 4 - 2 * (wtype == o.W_Q4_0):][:, :, :16]
        q = np.concatenate([qs & 15, qs >> 4], axis=2).astype(np.float64)
        if wtype == o.W_Q4_0:
            out = (q - 8) * h(b, 0)[..., None]
        else:
            out = q * h(b, 0)[..., None] + h(b, 2)[..., None]
        return out.reshape(n, K)
    if wtype == o.W_Q1_0:   # bit j of the 16 sign bytes, least significant first
        bits = np.unpackbits(b[:, :, 2:18], axis=2, bitorder="little").astype(np.float64)
        return ((2 * bits - 1) * h(b, 0)[..., None]).reshape(n, K)
    if wtype == o.W_PQ2_0:   # four 2-bit codes per byte, lowest first
        q = np.stack([(b[:, :, 2:34] >> (2 * i)) & 3 for i in range(4)], axis=3)
        return ((q.reshape(n, -1, 128).astype(np.float64) - 1) * h(b, 0)[..., None]).reshape(n, K)
    if wtype == o.W_PTQ1_0:
        # trit n of a byte = base-3 digit n (most significant first) of
        # floor(243 b / 256), the inverse of the encoder's ceil(256 q / 243)
        val = (b[:, :, 0:26].astype(np.int64) * 243) // 256
        dig = np.stack([(val // 3 ** (4 - i)) % 3 for i in range(5)], axis=3)   # (n, nb, 26, 5)
        t = np.zeros(b.shape[:2] + (128,), np.int64)
        for m in range(16):
            t[:, :, m + 16 * np.arange(5)] = dig[:, :, m, :]
        for m in range(8):
            t[:, :, 80 + m + 8 * np.arange(5)] = dig[:, :, 16 + m, :]
        for hh in range(2):
            t[:, :, 120 + hh + 2 * np.arange(4)] = dig[:, :, 24 + hh, :4]
        return ((t.astype(np.float64) - 1) * h(b, 26)[..., None]).reshape(n, K)
    if wtype == o.W_Q4_K:
        s = b[:, :, 4:16].astype(np.int64)
        sc = np.zeros(b.shape[:2] + (8,), np.int64)
        mn = np.zeros_like(sc)
        sc[..., :4] = s[..., 0:4] & 63
        mn[..., :4] = s[..., 4:8] & 63
        sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
        mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
        qs = b[:, :, 16:144].reshape(n, -1, 4, 32).astype(np.int64)
        q = np.stack([qs & 15, qs >> 4], axis=3).reshape(n, -1, 8, 32)   # sub-block = 2p + hi
        out = (h(b, 0)[..., None, None] * sc[..., None] * q
               - h(b, 2)[..., None, None] * mn[..., None])
        return out.reshape(n, K)
    # Q6_K
    ql = b[:, :, 0:128].reshape(n, -1, 2, 64).astype(np.int64)
    qh = b[:, :, 128:192].reshape(n, -1, 2, 32).astype(np.int64)
    lo = np.stack([ql[..., :32] & 15, ql[..., 32:] & 15, ql[..., :32] >> 4, ql[..., 32:] >> 4],
                  axis=3)                                            # (n, nb, half, quarter, 32)
    hi = np.stack([(qh >> (2 * t)) & 3 for t in range(4)], axis=3)
    q = (lo | (hi << 4)) - 32
    sc = b[:, :, 192:208].view(np.int8).astype(np.int64).reshape(n, -1, 2, 4, 2)
    scale = np.repeat(sc, 16, axis=4)                               # 16 weights per scale
    out = h(b, 208)[..., None, None, None] * scale * q
    return out.reshape(n, K)


# ---- packers written from the block layouts ---------------------------------

def pack_q4k(d, dmin, ls, lm, L):
    """ls, lm: 8 six-bit scales / mins; L: 256 four-bit quants (weight order)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = f16_bytes([d])
    blk[2:4] = f16_bytes([dmin])
    s = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            s[j] = ls[j]
            s[j + 4] = lm[j]
        else:
            s[j + 4] = (ls[j] & 15) | ((lm[j] & 15) << 4)
            s[j - 4] |= (ls[j] >> 4) << 6
            s[j] |= (lm[j] >> 4) << 6
    blk[4:16] = s
    for p in range(4):   # 64 weights per 32 bytes: low nibbles first
        blk[16 + 32 * p:16 + 32 * p + 32] = L[64 * p:64 * p + 32] | (L[64 * p + 32:64 * p + 64] << 4)
    return blk


def pack_q6k(d, scales, L):
    """scales: 16 int8, one per 16 consecutive weights; L: 256 six-bit quants."""
    blk = np.zeros(210, np.uint8)
    for n in range(2):
        q = L[128 * n:128 * n + 128]
        for l in range(32):
            q1, q2, q3, q4 = q[l], q[l + 32], q[l + 64], q[l + 96]
            blk[64 * n + l] = (q1 & 15) | ((q3 & 15) << 4)
            blk[64 * n + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            blk[128 + 32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = f16_bytes([d])
    return blk


def test_reference_golden_blocks():
    # test/gguf.test.ts:117-143
    q40 = np.array([0x00, 0x38] + [0x97] * 16, np.uint8)
    assert o.dequant_row(o.W_Q4_0, q40, 32).tolist() == [-0.5] * 16 + [0.5] * 16
    q41 = np.array([0x00, 0x38, 0x00, 0x3c] + [0x42] * 16, np.uint8)
    assert o.dequant_row(o.W_Q4_1, q41, 32).tolist() == [2.0] * 16 + [3.0] * 16


GOLDEN_BLOCKS = os.path.join(os.path.dirname(__file__), "golden", "ternary_blocks.json")


def _golden_blocks():
    with open(GOLDEN_BLOCKS) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden_blocks(), ids=lambda c: c["name"])
def test_reference_golden_128_blocks(case):
    """test/gguf.test.ts:32-124: Q1_0, PQ2_0 and PTQ1_0 (encoded by the
    test's own base-3 packer) decode to the test's weights."""
    B, _ = o.block_spec(case["type"])
    blk = np.array(case["block"], np.uint8)
    want = np.array(case["weights"], np.float32)
    assert np.array_equal(o.dequant_row(case["type"], blk, B), want)
    assert np.array_equal(np_weights(case["type"], blk.reshape(1, -1), B)[0], want)


def _dense_hadamard(n=512):
    # the reference test's dense Sylvester matrix: sign = parity of popcount(r & c)
    r = np.arange(n)[:, None] & np.arange(n)[None, :]
    par = np.zeros_like(r)
    for b in range(10):
        par ^= (r >> b) & 1
    return np.where(par == 1, -1.0, 1.0) / np.sqrt(n)


def test_hadamard_matches_dense_and_is_involutory():
    """test/gguf.test.ts:146-181: the fast rotation equals the dense
    Sylvester matrix product and applying it twice restores the input."""
    orig = (np.sin(np.arange(512) * 0.13) - 0.5).astype(np.float32)[None, :]
    H = _dense_hadamard()
    fast = o.hadamard512(orig)
    assert np.max(np.abs(fast[0] - H @ orig[0].astype(np.float64))) < 1e-5
    assert np.max(np.abs(o.hadamard512(fast) - orig)) < 1e-5


def test_hadamard_known_answers_and_signs():
    norm = np.float32(1 / np.sqrt(512))
    e0 = np.zeros((1, 1024), np.float32)
    e0[0, 0] = 1
    e0[0, 512 + 3] = 2                       # the second block is rotated on its own
    y = o.hadamard512(e0)
    assert np.all(y[0, :512] == norm)
    col = _dense_hadamard()[:, 3] * np.sqrt(512)   # +-1 column 3 of the unnormalised matrix
    assert np.array_equal(y[0, 512:], (2 * col).astype(np.float32) * norm)
    # integer inputs: every butterfly sum is exact, so only the norm rounds
    rng = np.random.default_rng(2)
    x = rng.integers(-1000, 1000, (3, 512)).astype(np.float32)
    want = (x.astype(np.float64) @ (_dense_hadamard() * np.sqrt(512)).T).astype(np.float32) * norm
    assert np.array_equal(o.hadamard512(x), want)
    # signs multiply the input first
    signs = np.where(rng.random(1024) < 0.5, -1.0, 1.0).astype(np.float32)
    x2 = rng.standard_normal((2, 1024)).astype(np.float32)
    assert np.array_equal(o.hadamard512(x2, signs), o.hadamard512(x2 * signs))


def test_fp16_every_pattern():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([o.fp16(int(v)) for v in h], np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


@pytest.mark.parametrize("wtype", TYPES + TERNARY)
def test_dequant_matches_numpy_decoder(wtype):
    rng = np.random.default_rng(wtype)
    K = 512
    w = random_blocks(wtype, 6, K, rng)
    want = np_weights(wtype, w, K)
    for r in range(6):
        got = o.dequant_row(wtype, w[r], K).astype(np.float64)
        # the reference dequantiser rounds products to binary32
        assert np.allclose(got, want[r], rtol=2 ** -22, atol=0), wtype


def test_q4k_layout_round_trip():
    rng = np.random.default_rng(3)
    for _ in range(20):
        ls, lm = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        L = rng.integers(0, 16, 256)
        d, dmin = 0.125, 0.0625     # powers of two: every product exact in binary32
        blk = pack_q4k(d, dmin, ls, lm, L)
        want = d * ls[np.arange(256) // 32] * L - dmin * lm[np.arange(256) // 32]
        assert o.dequant_row(o.W_Q4_K, blk, 256).tolist() == want.tolist()
        assert np_weights(o.W_Q4_K, blk.reshape(1, -1), 256)[0].tolist() == want.tolist()


def test_q6k_layout_round_trip():
    rng = np.random.default_rng(4)
    for _ in range(20):
        sc = rng.integers(-128, 128, 16)
        L = rng.integers(0, 64, 256)
        d = 0.25
        blk = pack_q6k(d, sc, L)
        want = d * sc[np.arange(256) // 16] * (L - 32)
        assert o.dequant_row(o.W_Q6_K, blk, 256).tolist() == want.tolist()
        assert np_weights(o.W_Q6_K, blk.reshape(1, -1), 256)[0].tolist() == want.tolist()


@pytest.mark.parametrize("wtype", TYPES + TERNARY)
def test_exact_gemv_matches_numpy(wtype):
    rng = np.random.default_rng(10 + wtype)
    K, N = 1024, 9
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((2, K)).astype(np.float32)
    y, mag = o.gemv_exact(wtype, x, w, N)
    W = np_weights(wtype, w, K)
    want = x.astype(np.float64) @ W.T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12 * np.abs(x.astype(np.float64)) @ np.abs(W).T)
    assert np.allclose(mag, np.abs(x.astype(np.float64)) @ np.abs(W).T, rtol=1e-12)


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("K", [256, 2048])
def test_reference_order_within_rounding_bound(wtype, K):
    rng = np.random.default_rng(K + wtype)
    N = 17
    w = random_blocks(wtype, N, K, rng)
    x = rng.standard_normal((1, K)).astype(np.float32)
    y, mag = o.gemv_exact(wtype, x, w, N)
    ref = o.gemv_ref(wtype, x, w, N).astype(np.float64)
    # binary32 sums of K terms: |err| <= about K * 2^-24 * sum |x w|; the
    # order of the reference (64 strided partial sums, then a tree) keeps it
    # far below that
    assert np.all(np.abs(ref - y) <= 2 ** -16 * mag + 1e-30)
    assert np.max(np.abs(ref - y) / mag) > 0   # binary32 rounding is visible
