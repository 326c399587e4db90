"""The row kernel's slot replay keeps, for k <= 64, each slot's rank among
the slots by (value, slot index) instead of searching for the minimum after
every entering logit (replay_row in hachiue_amd/csrc/sampler_kernels.hip).
This checks that bookkeeping, restated per lane, against the oracle's own
replace-min slot order (src/sampler.ts:50-69) on rows with many equal values
and signed zeros: the ids per slot must be identical."""
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
