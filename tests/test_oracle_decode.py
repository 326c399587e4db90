"""The decode-loop oracle (oracle/pyoracle.py decode_loop, src/engine.ts:
1626-1644) pinned on hand-worked sequences: greedy draws under a repetition
penalty whose 128-id window (src/sampler.ts:26) decides the answer, the stop
check before the history push, and rows that stay done."""
import numpy as np

from oracle import pyoracle as o

GREEDY_REP = dict(temperature=0.0, repetitionPenalty=4.0)


def steps(base, n, rows=1):
    return [np.tile(np.asarray(base, np.float32), (rows, 1)) for _ in range(n)]


def test_greedy_repetition_sequence():
    # logits [1, 2, 3, 0.5] each step, penalty 4: 3 -> 0.75 once 2 is in the
    # history, then 2 -> 0.5, then 1 -> 0.25; afterwards 2 (0.75) wins again
    res = o.decode_loop(steps([1, 2, 3, 0.5], 5), 4, [[]], [], [GREEDY_REP], [[0.5]] * 5)
    assert res.tokens[:, 0].tolist() == [2, 1, 0, 2, 2]
    assert res.histories[0] == [2, 1, 0, 2, 2]


def test_stop_id_ends_row_before_push():
    res = o.decode_loop(steps([1, 2, 3, 0.5], 5), 4, [[]], [0], [GREEDY_REP], [[0.5]] * 5)
    assert res.tokens[:, 0].tolist() == [2, 1, 0, -1, -1]
    assert res.histories[0] == [2, 1]
    assert res.done == [True]


def test_window_of_128():
    # id 2 sits 129 ids back: outside history.slice(-128), so not penalised
    prompt = [2] + [3] * 128
    res = o.decode_loop(steps([1, 2, 3, 0.5], 1), 4, [prompt], [], [GREEDY_REP], [[0.5]])
    assert res.tokens[0, 0] == 2
    prompt = [2] + [3] * 127      # 128 back: inside, penalised to 0.75
    res = o.decode_loop(steps([1, 2, 3, 0.5], 1), 4, [prompt], [], [GREEDY_REP], [[0.5]])
    assert res.tokens[0, 0] == 1


def test_ring_cap_truncates_frequency_counts():
    # frequency 1 per occurrence: id 2 seen 3 times -> 0, id 1 once -> 1
    cfg = dict(temperature=0.0, frequencyPenalty=1.0)
    prompt = [2, 2, 2, 1]
    full = o.decode_loop(steps([1, 2, 3, 0.5], 1), 4, [prompt], [], [cfg], [[0.5]])
    assert full.tokens[0, 0] == 0     # [1, 1, 0, 0.5]: first maximum is id 0
    # a ring of 2 keeps [2, 1]: [1, 1, 2, 0.5] -> id 2
    ring = o.decode_loop(steps([1, 2, 3, 0.5], 1), 4, [prompt], [], [cfg], [[0.5]], ring_cap=2)
    assert ring.tokens[0, 0] == 2


def test_rows_independent():
    cfgs = [GREEDY_REP, dict(temperature=0.0)]
    res = o.decode_loop(steps([1, 2, 3, 0.5], 3, rows=2), 4, [[], []], [1], cfgs,
                        [[0.5, 0.5]] * 3)
    assert res.tokens.tolist() == [[2, 2], [1, 2], [-1, 2]]
    assert res.histories == [[2], [2, 2, 2]]
