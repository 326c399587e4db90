"""GPU parity on the edge cases the reference's semantics single out
(src/sampler.ts): signed zeros, NaN / +-Infinity, ties at and inside the
top-k (slot-history order), k beyond the finite count, fractional / zero /
negative / infinite topK, NaN options, penalties below 1 and on zeros,
ragged vocab and stride, empty and out-of-range histories, extreme uniforms.
Both kernel routes (row kernel, chunk + finalize) are checked."""
import numpy as np
import pytest

from tests.gpu_util import compare, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def _batch(cases, vocab, stride=None):
    stride = stride or vocab
    rows = len(cases)
    logits = np.full((rows, stride), np.float32(np.nan), np.float32)
    hists, configs, us = [], [], []
    for r, (row, hist, cfg, u) in enumerate(cases):
        row = np.asarray(row, np.float32)
        logits[r, :row.size] = row
        hists.append(np.asarray(hist, np.int32))
        configs.append(cfg)
        us.append(u)
    off = np.zeros(rows + 1, np.int64)
    for r, h in enumerate(hists):
        off[r + 1] = off[r] + h.size
    ids = np.concatenate(hists).astype(np.int32) if off[-1] else np.zeros(1, np.int32)
    return logits, ids, off, configs, np.array(us, np.float64)


def _run(sampler, cases, vocab, stride=None, cap=64, label="edges", want_cands=True):
    logits, ids, off, configs, us = _batch(cases, vocab, stride)
    got = run_gpu(sampler, logits, vocab, ids, off, configs, us, cap, stride=logits.shape[1],
                  want_cands=want_cands)
    want, want_logits = run_oracle(logits, vocab, ids, off, configs, us, cap)
    compare(got, want, want_logits, configs, vocab, cap, label)
    return got, want


def _rng(seed):
    return np.random.default_rng(seed)


SAMPLE = dict(temperature=0.7, topK=40, topP=0.9)


def test_signed_zeros(any_sampler):
    V = 3000
    r = _rng(1)
    a = np.where(r.random(V) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
    b = a.copy(); b[:5] = -1.0
    c = -np.abs(r.standard_normal(V).astype(np.float32)); c[[7, 900, 2000]] = -0.0; c[50] = 0.0
    cases = [(a, [], SAMPLE, 0.3), (b, [], dict(temperature=0.0), 0.5),
             (c, [], dict(temperature=1.0, topK=3, topP=1.0), 0.9),
             (a, [], dict(temperature=1.0, topK=1), 0.2)]
    _run(any_sampler, cases, V)


def test_nan_and_infinities(any_sampler):
    V = 2000
    r = _rng(2)
    base = r.standard_normal(V).astype(np.float32)
    one_inf = base.copy(); one_inf[123] = np.inf
    two_inf = base.copy(); two_inf[[5, 1500]] = np.inf
    nan0 = base.copy(); nan0[0] = np.nan
    some_nan = base.copy(); some_nan[::7] = np.nan
    all_nan = np.full(V, np.nan, np.float32)
    all_ninf = np.full(V, -np.inf, np.float32)
    one_finite = all_ninf.copy(); one_finite[777] = 3.0
    ninf_mix = base.copy(); ninf_mix[::3] = -np.inf
    cases = [(one_inf, [], SAMPLE, 0.5), (two_inf, [], SAMPLE, 0.5),
             (nan0, [], dict(temperature=0.0), 0.1), (nan0, [], SAMPLE, 0.4),
             (some_nan, [], SAMPLE, 0.6), (all_nan, [], SAMPLE, 0.5),
             (all_nan, [], dict(temperature=0.0), 0.5), (all_ninf, [], SAMPLE, 0.5),
             (all_ninf, [], dict(temperature=0.0), 0.5), (one_finite, [], SAMPLE, 0.5),
             (ninf_mix, [], dict(temperature=0.9, topK=100, topP=0.95), 0.7)]
    _run(any_sampler, cases, V)


def test_ties(any_sampler):
    V = 5000
    r = _rng(3)
    all_eq = np.ones(V, np.float32)
    boundary = r.standard_normal(V).astype(np.float32)
    boundary[r.choice(V, 60, replace=False)] = 4.0          # 60 equal values around the k-th
    inside = r.standard_normal(V).astype(np.float32)
    inside[r.choice(V, 6, replace=False)] = 9.0             # a tie group at the top
    coarse = np.round(r.standard_normal(V) * 4).astype(np.float32)   # many duplicates
    kmax_tie = r.standard_normal(V).astype(np.float32); kmax_tie[[10, 20, 4000]] = 7.5
    cases = [(all_eq, [], SAMPLE, 0.5), (all_eq, [], dict(temperature=0.0), 0.5),
             (boundary, [], SAMPLE, 0.99), (inside, [], SAMPLE, 0.01),
             (inside, [], dict(temperature=1.0, topK=10, topP=1.0), 0.55),
             (coarse, [], dict(temperature=1.3, topK=64, topP=1.0), 0.77),
             (coarse, [], dict(temperature=1.3, topK=200, topP=1.0), 0.33),
             (kmax_tie, [], dict(temperature=1.0, topK=1), 0.5),
             (kmax_tie, [], dict(temperature=0.0), 0.5)]
    for u in (0.0, 0.25, 0.5, 0.75, 1.0 - 2.0 ** -53):
        cases.append((inside, [], dict(temperature=0.5, topK=8, topP=1.0), u))
    _run(any_sampler, cases, V, cap=256)


def test_k_beyond_finite_and_topk_forms(any_sampler):
    V = 50
    r = _rng(4)
    row = np.round(r.standard_normal(V) * 2).astype(np.float32)
    sparse = np.full(V, -np.inf, np.float32); sparse[[3, 9, 11, 30]] = [1.0, 2.0, 1.0, 2.0]
    cases = [(row, [], dict(temperature=1.0, topK=64, topP=1.0), 0.42),
             (row, [], dict(temperature=1.0, topK=float("inf"), topP=0.8), 0.42),
             (row, [], dict(temperature=1.0, topK=0), 0.3),        # 0 -> 64
             (row, [], dict(temperature=1.0, topK=-3), 0.3),       # negative -> 64
             (row, [], dict(temperature=1.0, topK=2.7), 0.6),      # truncated to 2
             (row, [], dict(temperature=1.0, topK=0.5), 0.6),      # max(1, 0.5) -> 1
             (row, [], dict(temperature=1.0, topK=float("nan")), 0.6),   # NaN -> 64
             (sparse, [], dict(temperature=1.0, topK=3, topP=1.0), 0.99),
             (sparse, [], dict(temperature=1.0, topK=10, topP=1.0), 0.99),
             (row, [], {}, 0.5)]                                   # reference defaults
    _run(any_sampler, cases, V)


def test_option_edge_values(any_sampler):
    V = 4000
    r = _rng(5)
    row = (r.standard_normal(V) * 2.5).astype(np.float32)
    cases = [(row, [], dict(temperature=float("nan")), 0.5),
             (row, [], dict(temperature=0.7, topP=float("nan")), 0.5),
             (row, [], dict(temperature=0.7, minP=float("nan")), 0.5),
             (row, [], dict(temperature=0.7, minP=0.05), 0.8),
             (row, [], dict(temperature=0.7, minP=1.0), 0.8),
             (row, [], dict(temperature=0.7, minP=2.0), 0.8),
             (row, [], dict(temperature=0.7, topP=0.0), 0.8),
             (row, [], dict(temperature=1e-6, topK=40), 0.8),
             (row, [], dict(temperature=1e6, topK=40, topP=0.5), 0.8),
             (row, [], dict(temperature=-1.0), 0.8),
             (row, [], dict(temperature=0.7, topK=40, topP=0.9), 0.0),
             # probabilities below 2^-29 among the candidates: the tail's
             # cumulative sums take the sequential path
             (row, [], dict(temperature=0.1, topK=60, topP=1.0), 0.9999999),
             (row, [], dict(temperature=0.12, topK=64, topP=0.9999999), 0.999),
             (row, [], dict(temperature=0.09, topK=64, topP=1.0, minP=1e-12), 0.5)]
    _run(any_sampler, cases, V)


def test_penalty_edges(any_sampler):
    V = 6000
    r = _rng(6)
    row = (r.standard_normal(V) * 2).astype(np.float32)
    row[[10, 11, 12]] = [0.0, -0.0, -3.0]
    long_hist = [7] + list(r.integers(0, V, 128))                  # id 7 falls out of the last 128
    cases = [(row, [10, 11, 12, 12, 12, -5, V, V + 3, 2**31 - 1], dict(repetitionPenalty=2.0, **SAMPLE), 0.4),
             (row, [10, 11, 12], dict(repetitionPenalty=0.8, **SAMPLE), 0.4),
             (row, [10, 11, 12, 100], dict(repetitionPenalty=0.0, **SAMPLE), 0.4),
             (row, [10, 100], dict(repetitionPenalty=float("nan"), **SAMPLE), 0.4),
             (row, long_hist, dict(repetitionPenalty=1.3, **SAMPLE), 0.4),
             (row, [], dict(repetitionPenalty=1.3, **SAMPLE), 0.4),
             (row, list(r.integers(0, 50, 300)), dict(repetitionPenalty=1.2, presencePenalty=0.5,
                                                      frequencyPenalty=0.25, **SAMPLE), 0.4),
             (row, [5, 5, 5, 9], dict(presencePenalty=-1.0, frequencyPenalty=0.0, **SAMPLE), 0.4),
             (row, [5, 5, 5, 9], dict(temperature=0.0, repetitionPenalty=1.5), 0.4)]
    _run(any_sampler, cases, V)


def test_penalty_history_beyond_the_table(any_sampler):
    """Histories whose distinct ids exceed the pre-pass's LDS hash table
    (8192 slots) are counted by id ranges instead; one with few distinct ids
    but long, and one hot id repeated thousands of times."""
    V = 40000
    r = _rng(8)
    row = (r.standard_normal(V) * 2).astype(np.float32)
    many = list(r.integers(0, V, 20000))                   # ~15k distinct ids
    hot = [123] * 3000 + list(r.integers(0, 64, 3000))     # few distinct, long
    pf = dict(presencePenalty=0.4, frequencyPenalty=0.05, **SAMPLE)
    cases = [(row, many, dict(repetitionPenalty=1.2, **pf), 0.3),
             (row, many, pf, 0.6),
             (row, hot, dict(repetitionPenalty=1.1, **pf), 0.5),
             (row, many, dict(temperature=1.0, topK=5000, topP=0.9, repetitionPenalty=1.3), 0.7),
             (row, many, dict(temperature=0.0, presencePenalty=0.3), 0.5)]
    _run(any_sampler, cases, V)


@pytest.mark.parametrize("stride", [151940, 151937])
def test_mid_penalties_long_histories(any_sampler, stride):
    """Presence / frequency rows of the mid kernel (64 < k <= 1024).  The
    history is counted while the first rounds load, its ids are left out of
    the stream's counts and their penalised logits joined at the end, unless
    its distinct ids overflow the list (2048) or the table (then counted by
    id ranges): that row is rewritten in place and read again.  Short and
    long histories, repeated ids.
    The histories hit the row's top logits (in round 0, later rounds and the
    last logit past the whole float4s), so the penalties change the candidate
    set.  Aligned rows (the last logit read apart from the float4s) and
    unaligned ones.  Candidate ids, probabilities and penalised logits
    against the oracle."""
    V = 151937
    r = _rng(21)
    row = (r.standard_normal(V) * 2.5).astype(np.float32)
    row[V - 1] = 11.0
    row[100] = 10.5                                       # in round 0
    top = [int(i) for i in np.argsort(-row)[:1500]]
    short = top[:300] + list(r.integers(0, V, 1200))      # 1500 entries
    listed = list(r.choice(top, 3000)) + [V - 1, 100]     # > 2048 entries, <= 1500 distinct
    over_list = [int(i) for i in r.choice(V, 4000, replace=False)] + top[:600] * 2
    over_table = list(r.integers(0, V, 20000)) + top[:200]
    pf = dict(temperature=0.8, topK=300, topP=0.95, presencePenalty=0.5, frequencyPenalty=0.2)
    cases = [(row, short, pf, 0.3),
             (row, listed, pf, 0.6),
             (row, listed, dict(pf, repetitionPenalty=1.3, topK=1000, topP=0.99), 0.9),
             (row, over_list, pf, 0.45),
             (row, over_table, dict(pf, repetitionPenalty=1.1), 0.2),
             (row, listed, dict(temperature=0.0, presencePenalty=2.0, frequencyPenalty=0.1), 0.5)]
    _run(any_sampler, cases, V, stride=stride, cap=1024, label="mid penalties")


@pytest.mark.parametrize("vocab,pad", [(151669, 0), (1001, 3), (4097, 1), (1, 0), (2, 5), (3, 0),
                                       (151937, 3), (50257, 3), (32003, 1), (6, 2), (7, 1)])
def test_ragged_vocab_and_stride(any_sampler, vocab, pad):
    """Rows whose length is not a multiple of four, with 16-byte aligned
    strides (the last logits lie past the last whole float4) and unaligned
    ones.  The last logits of some rows are planted as the largest, one of
    them also in the repetition history."""
    r = _rng(vocab + pad)
    cases = []
    for i in range(3):
        row = (r.standard_normal(vocab) * 2).astype(np.float32)
        hist = list(r.integers(0, vocab, 20))
        cases.append((row, hist, dict(temperature=0.8, topK=40, topP=0.95, repetitionPenalty=1.1),
                      float(r.random())))
    cases.append((cases[0][0], [], dict(temperature=0.0), 0.5))
    top = (r.standard_normal(vocab) * 2).astype(np.float32)
    top[-3:] = np.float32([9.0, 9.5, 10.0])[-min(3, vocab):]
    cases.append((top, [], dict(temperature=0.0), 0.5))
    cases.append((top, [vocab - 1], dict(temperature=1.0, topK=5, topP=1.0,
                                         repetitionPenalty=1.5), 0.999))
    cases.append((top, [vocab - 1], dict(temperature=0.0, repetitionPenalty=100.0), 0.5))
    _run(any_sampler, cases, vocab, stride=vocab + pad)


def test_mid_k_tail_without_candidate_outputs(any_sampler):
    """Rows with 64 < k <= 1024 and no candidate outputs: the block-parallel
    tail (exact prefix sums over the sorted list) and its sequential
    fallbacks (ties at or inside the top k, probabilities below 2^-29, u = 0,
    min-p and top-p edges, an infinite logit)."""
    V = 30000
    r = _rng(12)
    base = (r.standard_normal(V) * 2.5).astype(np.float32)
    ties = base.copy()
    top = np.argsort(-base)[:300]
    ties[top[10:20]] = ties[top[10]]          # a tie group inside the top k
    ties[top[199:230]] = ties[top[199]]       # a group at the k-th value (k = 200)
    inf = base.copy(); inf[777] = np.inf
    cases = [(base, [], dict(temperature=0.8, topK=300, topP=0.9), 0.37),
             (base, [], dict(temperature=1.5, topK=1024, topP=0.99), 0.61),
             (base, [], dict(temperature=0.05, topK=500, topP=0.95), 0.5),    # tiny probabilities
             (base, [], dict(temperature=1.0, topK=100, topP=0.0), 0.5),
             (base, [], dict(temperature=1.0, topK=100, topP=1.0), 0.999),
             (base, [], dict(temperature=1.0, topK=100, topP=0.9, minP=0.3), 0.7),
             (base, [], dict(temperature=1.0, topK=100, topP=0.9, minP=1.0), 0.7),
             (base, [], dict(temperature=1.0, topK=100, topP=0.9), 0.0),
             (ties, [], dict(temperature=1.0, topK=200, topP=0.95), 0.42),
             (ties, [], dict(temperature=3.0, topK=200, topP=1.0), 0.999999),
             (inf, [], dict(temperature=1.0, topK=100, topP=0.9), 0.5),
             (base, list(r.integers(0, V, 100)), dict(temperature=0.9, topK=80, topP=0.9,
                                                     repetitionPenalty=1.2), 0.25)]
    _run(any_sampler, cases, V, cap=1024, label="mid-k tokens only", want_cands=False)


@pytest.mark.parametrize("k", [40, 500])
def test_every_logit_enters_the_candidate_lists(any_sampler, k):
    """Full-size rows on which every logit of the stream passes the bound:
    all equal, and increasing with the index (each round lies above every
    bound taken before it).  The per-wave candidate segments overflow, the
    row goes to the slot replay, and the repetition write-back touches the
    first and the last id of the row."""
    V = 151936
    eq = np.ones(V, np.float32)
    inc = (np.arange(V, dtype=np.float32) * np.float32(1e-3)).astype(np.float32)
    edge = [0, V - 1, 1, V - 2, V - 1]
    cfg = dict(temperature=0.7, topK=k, topP=0.9)
    rep = dict(repetitionPenalty=1.3, **cfg)
    cases = [(eq, [], cfg, 0.5), (eq, edge, rep, 0.25), (inc, [], cfg, 0.6),
             (inc, edge, rep, 0.9), (inc, edge, dict(temperature=0.0, repetitionPenalty=1.3), 0.5),
             (eq, edge, dict(temperature=1.0, topK=k, topP=1.0, repetitionPenalty=0.5), 0.999)]
    _run(any_sampler, cases, V, cap=64, label=f"every logit enters, k={k}")


@pytest.mark.parametrize("k", [1, 3, 40, 64])
def test_slot_replay_full_rows(any_sampler, k):
    """Full-vocabulary rows whose draw falls in a group of equal logits: at
    the top, inside the top-k, and at the k-th largest with copies before and
    after it; one row also with the repetition penalty, one rising through
    the row (every block can hold a logit that enters).  The replace-min scan
    decides the order inside the group (src/sampler.ts:50-74), and the
    candidate ids must follow it.  On the row kernel this is the staged
    replay: one wave lists the blocks that can hold an entering logit, the
    others copy them into LDS, a third wave scans them."""
    V = 151936
    r = _rng(40 + k)
    base = r.standard_normal(V).astype(np.float32)
    o = np.argsort(-base, kind="stable")
    top = base.copy()
    top[o[min(3, k)]] = top[o[0]]                  # the largest twice
    inner = base.copy()
    inner[o[k // 2]] = inner[o[max(0, k // 2 - 1)]]  # an equal pair inside the top-k
    kth = base.copy()
    kth[r.choice(V, 5, replace=False)] = kth[o[k - 1]]   # copies of the k-th largest
    rise = (np.arange(V, dtype=np.float32) * np.float32(1e-4) +
            r.integers(0, 3, V).astype(np.float32)).astype(np.float32)
    hist = list(o[:3]) + list(r.integers(0, V, 20))
    cfg = dict(temperature=0.7, topK=k, topP=1.0)
    cases = [(top, [], cfg, 1e-4), (inner, [], cfg, 0.5), (kth, [], cfg, 0.999),
             (kth, hist, dict(repetitionPenalty=1.2, **cfg), 0.3), (rise, [], cfg, 0.7),
             (top, [], dict(temperature=0.0, topK=k), 0.5)]
    got, _ = _run(any_sampler, cases, V, cap=64, label=f"slot replay, full rows, k={k}")
    if k > 1:   # candidate outputs and a tie inside the top-k: the replay ran (HS_ROW_REPLAYED)
        assert got.flags[0] & 0x2 and got.flags[1] & 0x2, got.flags


@pytest.mark.parametrize("k", [2, 40, 64])
def test_slot_replay_ragged_rows(any_sampler, k):
    """The staged replay on rows that are not 16-byte aligned (stride V + 1,
    V not a multiple of 4 or 64), whose first k logits hold -Infinity or NaN
    (no sorted fill: the slots fill by insertion), and with fewer finite
    logits than k after the first block."""
    V = 150001
    r = _rng(70 + k)
    base = r.standard_normal(V).astype(np.float32)
    o = np.argsort(-base, kind="stable")
    top = base.copy()
    top[o[min(2, k - 1)]] = top[o[0]]                    # the largest twice (k >= 2)
    holes = top.copy()
    holes[[0, 3, k // 2]] = -np.inf
    holes[5] = np.nan
    sparse = np.full(V, -np.inf, np.float32)
    sparse[r.choice(V, k + 3, replace=False)] = r.integers(0, 3, k + 3).astype(np.float32)
    cfg = dict(temperature=0.8, topK=k, topP=1.0)
    cases = [(top, [], cfg, 1e-4), (holes, [], cfg, 1e-4), (sparse, [], cfg, 0.6),
             (holes, list(o[:4]), dict(repetitionPenalty=1.3, **cfg), 0.2)]
    _run(any_sampler, cases, V, stride=V + 1, cap=64, label=f"slot replay, ragged rows, k={k}")
