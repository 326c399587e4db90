"""Loader of the hand-traced known-answer cases (tests/golden/sampler_kat.json)."""
import json
import math
import os

import numpy as np

PATH = os.path.join(os.path.dirname(__file__), "golden", "sampler_kat.json")

_SPECIAL = {"NaN": float("nan"), "Infinity": float("inf"), "-Infinity": float("-inf"),
            "-0": -0.0}


def num(x):
    return _SPECIAL[x] if isinstance(x, str) else float(x)


def f32_array(xs):
    return np.array([num(x) for x in xs], dtype=np.float32)


def config(c):
    return {k: num(v) for k, v in c.items()}


def load():
    with open(PATH) as f:
        return json.load(f)


def cases():
    return load()["cases"]


def same_f32(a, b):
    """Bitwise equality of float32 arrays (so -0 differs from 0, NaN == NaN)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def rep_closed(logits, history, vocab, p):
    """Closed form of the repetition step for the greedy_sees_penalty case:
    each distinct in-range id of the last 128 entries, v<0 ? v*p : v/p,
    rounded to float32 (IEEE binary64 arithmetic is exact-rounded, so this
    is fixed by the mathematics, not by an implementation)."""
    out = np.array(logits, np.float32)
    for i in set(history[-128:]):
        if 0 <= i < vocab:
            v = float(out[i])
            out[i] = np.float32(v * p if v < 0 else v / p)
    return out


def is_nan(x):
    return isinstance(x, float) and math.isnan(x)
