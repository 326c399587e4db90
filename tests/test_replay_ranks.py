"""The row kernel's slot replay (replay_row in
hachiue_amd/csrc/sampler_kernels.hip) keeps, for k <= 64, the k slots in the
lanes of one wave sorted by (value, slot index): lane 0 holds the slot the
reference's rescan finds (the first slot holding the minimum).  An entering
logit takes lane 0's slot; its position p is the number of other slots below
it, lanes 1..p move down one lane (a wave shift) and the new slot goes to
lane p.  An earlier form kept each slot in its own lane with its rank.  The
current form (LaneSlots, and PackedSlots with the logit index inside a
complemented 64-bit word) needs no count: lane j takes min(c[j + 1],
max(c[j], c')), which leaves every lane as it is for a logit that does not
enter, so the kernel applies it to every candidate without a test.  The
staged replay lists the 64-logit blocks whose largest key is above the k-th
largest of the earlier blocks' largest keys.  Each is restated per lane here
and checked against the oracle's own replace-min slot order
(src/sampler.ts:50-69) on rows with many equal values, signed zeros and NaN:
the ids per slot must be identical, and every block holding a logit that
enters must be listed."""
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



def f2key(x: np.ndarray) -> np.ndarray:
    """The kernels' order-preserving key of a binary32 logit: -0 == +0, and
    NaN and -Infinity (which never enter) are 0."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = np.where(u == 0x80000000, 0, u)
    k = np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    return np.where(np.asarray(x, np.float32) > -np.inf, k, 0).astype(np.uint64)


def minmax_replay(x: np.ndarray, k: int, packed: bool, fill: bool = False):
    """LaneSlots (packed=False: c = key << 32 | slot, the index in its own
    lane) or PackedSlots (packed=True: ~(key << 32 | slot << 20 | index),
    compared without the index), updated for every logit with a key.  With
    fill (PackedSlots::scan_memory from the row's start), when the first k
    logits all have keys the lanes start as those k words sorted, and the
    scan starts at logit k."""
    M = (1 << 64) - 1
    NOI = 0xFFFFF
    lanes = np.arange(64)
    keys = f2key(x)
    if packed:
        c = [M & ~((j << 20) | NOI) if j < k else 0 for j in range(64)]
    else:
        c = [j if j < k else M for j in range(64)]
    rid = [-1] * 64
    start = 0
    if fill and packed and len(keys) >= k and all(int(v) != 0 for v in keys[:k]):
        words = sorted(M & ~((int(keys[j]) << 32) | (j << 20) | j) for j in range(k))[::-1]
        c = words + [0] * (64 - k)
        start = k
    for i, kx in enumerate(keys.tolist()):
        if kx == 0 or i < start:
            continue
        if packed:
            klo = (c[0] & 0xFFFFFFFF) | NOI                   # lane 0's low word, index bits set
            hi = ((~kx) & 0xFFFFFFFF) << 32
            cK = hi | klo
            cL = hi | (klo ^ i)
            nx = c[1:] + [0]                                  # lane 63 reads 0
            below = [cj > cK for cj in c]
            shift = [nj > cK for nj in nx]
        else:
            mi = c[0] & 0xFFFFFFFF
            cK = cL = (kx << 32) | mi
            nx = c[1:] + [M]                                  # lane 63 reads ~0
            below = [cj < cK for cj in c]
            shift = [nj < cK for nj in nx]
            nr = rid[1:] + [-1]
            rid = [nr[j] if shift[j] else (i if below[j] else rid[j]) for j in lanes]
        c = [nx[j] if shift[j] else (cL if below[j] else c[j]) for j in lanes]
    out = np.full(k, -1)
    for j in range(k):
        if packed:
            v = M & ~c[j]
            slot, ix = (v >> 20) & 63, v & NOI
            out[slot] = -1 if ix == NOI else ix
        else:
            out[c[j] & 0xFFFFFFFF] = rid[j]
    return out


def ordered_positions(lanes_asc):
    """PackedSlots::store_ordered on lanes sorted ascending by (key, slot):
    lane j goes to (k - 1 - last lane of its key's run) + (j - first lane)."""
    k = len(lanes_asc)
    keys = [kk for kk, _ in lanes_asc]
    runs = [j for j in range(k) if j == 0 or keys[j] != keys[j - 1]]
    pos = []
    for j in range(k):
        first = max(r for r in runs if r <= j)
        above = [r for r in runs if r > j]
        last = above[0] - 1 if above else k - 1
        pos.append((k - 1 - last) + (j - first))
    return pos


def listed_blocks(x: np.ndarray, k: int):
    """The staged replay's block list: the k largest block keys so far in
    lanes (ascending, min(r[j + 1], max(r[j], key)) per block), a block
    listed when its key is above lane 0's when it comes."""
    keys = f2key(x)
    nb = (len(x) + 63) // 64
    bkey = [int(keys[64 * b:64 * b + 64].max()) for b in range(nb)]
    r = [0 if j < k else 0xFFFFFFFF for j in range(64)]
    out = []
    for b, kb in enumerate(bkey):
        if kb > r[0]:
            out.append(b)
        nx = r[1:] + [0xFFFFFFFF]
        r = [min(nx[j], max(r[j], kb)) for j in range(64)]
    return set(out)


def entering(x: np.ndarray, k: int):
    """Indices that enter the reference's slots (src/sampler.ts:55-56)."""
    vals = [-np.inf] * k
    out = []
    for i, v in enumerate(np.asarray(x, np.float64)):
        mv = min(vals)
        if v > mv:
            vals[vals.index(mv)] = v
            out.append(i)
    return out


def _rows(rng):
    for _ in range(6):
        k = int(rng.integers(1, 65))
        n = int(rng.integers(1, 700))
        kind = rng.random()
        if kind < 0.4:
            x = (rng.integers(-12, 12, n) / 4).astype(np.float32)   # many ties
        elif kind < 0.7:
            x = rng.standard_normal(n).astype(np.float32)
        else:
            x = (np.arange(n) * 1e-3 + rng.integers(0, 3, n)).astype(np.float32)   # rising
        x[rng.integers(0, n, 3)] = np.float32(-0.0)
        if rng.random() < 0.3:
            x[rng.integers(0, n, 5)] = np.float32(np.nan)
        if rng.random() < 0.2:
            x[rng.integers(0, n, 5)] = -np.inf
        yield k, n, x


@pytest.mark.parametrize("seed", range(10))
@pytest.mark.parametrize("packed,fill", [(False, False), (True, False), (True, True)])
def test_minmax_lanes_match_slot_scan(seed, packed, fill):
    rng = np.random.default_rng(300 + seed)
    for k, n, x in _rows(rng):
        ids, _ = o.topk_slots(x, n, k)
        assert minmax_replay(x, k, packed, fill).tolist() == list(ids), (seed, k, n, packed, fill)


@pytest.mark.parametrize("seed", range(10))
def test_listed_blocks_hold_every_entering_logit(seed):
    rng = np.random.default_rng(400 + seed)
    for k, n, x in _rows(rng):
        need = {i // 64 for i in entering(x, k)}
        assert need <= listed_blocks(x, k), (seed, k, n)


@pytest.mark.parametrize("seed", range(8))
def test_ordered_store_is_the_stable_sort(seed):
    """The positions store_ordered gives the final slots equal the
    reference's order (src/sampler.ts:72-74): the slots sorted by value
    descending, equal values by slot ascending, empty slots (-Infinity) last."""
    rng = np.random.default_rng(500 + seed)
    for k, n, x in _rows(rng):
        ids, vals = o.topk_slots(x, n, k)
        keys = [int(f2key(np.float32(v))) if i >= 0 else 0 for i, v in zip(ids, vals)]
        lanes = sorted((keys[s], s) for s in range(k))          # ascending (key, slot)
        pos = ordered_positions(lanes)
        got = [None] * k
        for (kk, slot), p in zip(lanes, pos):
            got[p] = slot
        want = sorted(range(k), key=lambda s: (-keys[s], s))      # stable, value descending
        assert got == want, (seed, k, n)
