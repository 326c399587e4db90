"""The row kernel's slot replay (replay_row in
hachiue_amd/csrc/sampler_kernels.hip) keeps, for k <= 64, the k slots in the
lanes of one wave sorted by (value, slot index): lane 0 holds the slot the
reference's rescan finds (the first slot holding the minimum).  An entering
logit takes lane 0's slot; its position p is the number of other slots below
it, lanes 1..p move down one lane (a wave shift) and the new slot goes to
lane p.  An earlier form kept each slot in its own lane with its rank.  Both
are restated per lane here and checked against the oracle's own replace-min
slot order (src/sampler.ts:50-69) on rows with many equal values and signed
zeros: the ids per slot must be identical."""
import numpy as np
import pytest

from oracle import pyoracle as o


def rank_replay(x: np.ndarray, k: int):
    lanes = np.arange(64)
    rv = np.where(lanes < k, -np.inf, np.inf)
    rid = np.full(64, -1)
    rk = np.where(lanes < k, lanes, 64)
    mi, mv = 0, -np.inf
    for i, v in enumerate(x):
        if not v > mv:
            continue
        less = (lanes < k) & (lanes != mi) & ((rv < v) | ((rv == v) & (lanes < mi)))
        r = int(less.sum())                       # the entering logit's rank
        shift = (lanes != mi) & (rk >= 1) & (rk <= r)
        rk = np.where(shift, rk - 1, rk)
        rv[mi], rid[mi], rk[mi] = v, i, r
        mi = int(np.flatnonzero((lanes < k) & (rk == 0))[0])
        mv = rv[mi]
    return rid[:k]


def sorted_replay(x: np.ndarray, k: int):
    lanes = np.arange(64)
    rv = np.where(lanes < k, -np.inf, np.inf)   # value per lane, ascending
    rs = lanes.copy()                            # its slot
    rid = np.full(64, -1)                        # its logit index
    mv, ms = -np.inf, 0                          # lane 0: the minimum and its slot
    for i, v in enumerate(x):
        if not v > mv:
            continue
        less = (lanes >= 1) & (lanes < k) & ((rv < v) | ((rv == v) & (rs < ms)))
        p = int(less.sum())
        nv, ns, ni = np.roll(rv, -1), np.roll(rs, -1), np.roll(rid, -1)   # lane j <- lane j + 1
        low = lanes < p
        rv, rs, rid = np.where(low, nv, rv), np.where(low, ns, rs), np.where(low, ni, rid)
        rv[p], rs[p], rid[p] = v, ms, i
        mv, ms = rv[0], int(rs[0])
    out = np.full(k, -1)
    out[rs[:k]] = rid[:k]
    return out


@pytest.mark.parametrize("seed", range(12))
def test_sorted_lanes_match_slot_scan(seed):
    rng = np.random.default_rng(100 + seed)
    for _ in range(8):
        k = int(rng.integers(1, 65))
        n = int(rng.integers(1, 400))
        if rng.random() < 0.5:
            x = (rng.integers(-12, 12, n) / 4).astype(np.float32)   # many ties
        else:
            x = rng.standard_normal(n).astype(np.float32)
        x[rng.integers(0, n, 3)] = np.float32(-0.0)
        if rng.random() < 0.3:
            x[rng.integers(0, n, 5)] = np.float32(np.nan)
        ids, _ = o.topk_slots(x, n, k)
        want = np.asarray(ids)
        assert sorted_replay(x.astype(np.float64), k).tolist() == want.tolist(), (seed, k, n)


@pytest.mark.parametrize("seed", range(12))
def test_rank_bookkeeping_matches_slot_scan(seed):
    rng = np.random.default_rng(seed)
    for _ in range(8):
        k = int(rng.integers(1, 65))
        n = int(rng.integers(1, 400))
        if rng.random() < 0.5:
            x = (rng.integers(-12, 12, n) / 4).astype(np.float32)   # many ties
        else:
            x = rng.standard_normal(n).astype(np.float32)
        x[rng.integers(0, n, 3)] = np.float32(-0.0)
        ids, _ = o.topk_slots(x, n, k)
        want = np.asarray(ids)
        assert rank_replay(x.astype(np.float64), k).tolist() == want.tolist(), (seed, k, n)
