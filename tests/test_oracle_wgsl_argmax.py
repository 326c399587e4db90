"""The oracle's step-by-step simulation of the WGSL argmax
(src/kernels.ts:1613-1654), which the engine's GPU greedy route uses
(src/engine.ts:1600-1601), pinned against hand-derived answers of the
reduction tree and against an independent closed form:

    among the ids whose value is the maximum of the values > f32(-1e30),
    the winner has the smallest bit-reversed low byte (the invocation the
    tree prefers: at stride s, slot t keeps its value against slot t+s on a
    tie, so bit 7 of the invocation is decided first and bit 0 last), then
    the smallest id within that invocation's strided scan; 0 when no value
    exceeds f32(-1e30).
"""
import numpy as np
import pytest

from oracle import pyoracle

FLOOR = np.float32(-1e30)


def brev8(x):
    x = np.asarray(x, np.uint32) & 0xFF
    r = np.zeros_like(x)
    for b in range(8):
        r |= ((x >> b) & 1) << (7 - b)
    return r


def closed_form(row):
    v = np.asarray(row, np.float32)
    ok = v > FLOOR                       # NaN compares false
    if not ok.any():
        return 0
    m = v[ok].max()
    ids = np.nonzero(ok & (v == m))[0]   # -0 == +0
    key = brev8(ids).astype(np.int64) * (1 << 32) + (ids >> 8)
    return int(ids[np.argmin(key)])


def wgsl(row):
    row = np.asarray(row, np.float32)
    return int(pyoracle.wgsl_argmax(row.reshape(1, -1), row.size)[0])


def row_with(n, fill, **at):
    r = np.full(n, np.float32(fill), np.float32)
    for k, v in at.items():
        r[int(k[1:])] = v
    return r


# Hand-derived through the tree (stride 128, 64, ..., 1; ties keep the lower slot).
KATS = [
    ("unique maximum", row_with(2000, -1.0, i1000=3.0), 1000),
    # invocations 1 and 128: at stride 128 slot 0 takes 128's value (0's is
    # smaller); slot 1 keeps invocation 1's; at stride 1 they tie and slot 0
    # (invocation 128) is kept.  sampleLogits' argmax returns 1 here.
    ("ties at ids 1 and 128", row_with(300, -1.0, i1=7.0, i128=7.0), 128),
    # invocations 3 and 5: stride 4 moves 5 into slot 1, stride 2 keeps slot 1
    # against slot 3 on the tie, stride 1 moves slot 1 into slot 0.
    ("ties at ids 3 and 5", row_with(300, -1.0, i3=7.0, i5=7.0), 5),
    # one invocation (0) sees both: strict '>' keeps the first
    ("ties at ids 0 and 256", row_with(600, -1.0, i0=7.0, i256=7.0), 0),
    # invocation 0 (id 256) and invocation 1 (id 1) tie at stride 1: slot 0 kept
    ("ties at ids 256 and 1", row_with(600, -1.0, i1=7.0, i256=7.0), 256),
    # +0 at id 1 and -0 at id 2 are equal under '>': invocation 2 reaches slot 0
    # at stride 2 and keeps it against slot 1 at stride 1
    ("signed zeros", row_with(300, -1.0, i1=0.0, i2=-0.0), 2),
    ("all NaN", np.full(500, np.nan, np.float32), 0),
    ("all -Infinity", np.full(500, -np.inf, np.float32), 0),
    ("all at the initial value", np.full(500, FLOOR, np.float32), 0),
    # values at or below f32(-1e30) are never taken, -5e29 is
    ("below the initial value", row_with(500, -2e30, i7=-5e29), 7),
    # sampleLogits returns 0 here (its running maximum starts at logits[0] = NaN)
    ("NaN at id 0", row_with(500, 1.0, i0=np.nan, i321=2.0), 321),
    ("+Infinity", row_with(500, 1.0, i77=np.inf, i400=np.inf), 400),
]


@pytest.mark.parametrize("name,row,want", KATS, ids=[k[0] for k in KATS])
def test_known_answers(name, row, want):
    assert wgsl(row) == want
    assert closed_form(row) == want


def test_empty_row():
    assert int(pyoracle.wgsl_argmax(np.zeros((1, 4), np.float32), 0)[0]) == 0


@pytest.mark.parametrize("vocab", [1, 2, 3, 255, 256, 257, 511, 1000, 4099, 70001])
@pytest.mark.parametrize("kind", ["coarse", "specials", "normal"])
def test_simulation_equals_closed_form(vocab, kind):
    r = np.random.default_rng(vocab * 7 + len(kind))
    rows = []
    for _ in range(8):
        if kind == "coarse":        # many ties at the maximum
            row = r.integers(-3, 2, vocab).astype(np.float32)
        elif kind == "specials":
            row = r.choice(np.float32([np.nan, -np.inf, np.inf, 0.0, -0.0, 1.0, -2e30, FLOOR]),
                           vocab)
        else:
            row = (r.standard_normal(vocab) * 3).astype(np.float32)
        rows.append(row)
    x = np.stack(rows)
    got = pyoracle.wgsl_argmax(x, vocab)
    assert got.tolist() == [closed_form(row) for row in rows]


def test_unique_maximum_is_the_textbook_argmax():
    r = np.random.default_rng(5)
    for vocab in (17, 256, 151936):
        x = (r.standard_normal((4, vocab)) * 2).astype(np.float32)
        got = pyoracle.wgsl_argmax(x, vocab)
        assert got.tolist() == np.argmax(x, axis=1).tolist()


def test_strided_rows():
    r = np.random.default_rng(9)
    x = r.integers(-2, 3, (5, 1030)).astype(np.float32)
    got = pyoracle.wgsl_argmax(x, 1000, rows=5, stride=1030)
    assert got.tolist() == [closed_form(row[:1000]) for row in x]
