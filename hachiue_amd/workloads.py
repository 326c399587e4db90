"""Seeded synthetic sampling workloads.

Each workload is a batch of logit rows with per-row histories, sampling
options and uniforms, following the shapes and distributions of the
reference's sampling use (sampleLogits is called once per decode step with
the full token history, src/engine.ts:1642):

  single      1 x 151936, N(0, 2.5^2) + 8 spikes of +12 at seeded ids,
              repetition 1.1 over 64 uniform ids, T 0.7, k 40, p 0.9
              (greedy variant: T 0)
  batch64     64 x 151936, same logits, 256-token histories drawn from a
              small pool (repeats), repetition 1.1, T 0.8, k 40, p 0.95
  perrow256   256 x 151936, per-row k ~ U{1..1024}, p ~ U[0.5, 0.99],
              T ~ U[0.3, 1.5], presence 0.5, frequency 0.3 over 1024-token
              Zipf(1.1) histories
  gumbel1024  1024 x 151936 standard-Gumbel logits, top-p 0.98, k = vocab,
              T 1.0, no penalties
  v262k512    512 x 262144, N(0, 3^2), 4096-token Zipf(1.1) histories,
              repetition 1.15, presence 0.4, frequency 0.2, T 0.9, k 100,
              p 0.9
  headline    256 x 151936 with the `single` options per row (k 40, p 0.9,
              repetition 1.1 over 64 ids, T 0.7): the benchmark workload

`rows` / `vocab` overrides shrink a workload for quick tests while keeping
its distributions.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

from dataclasses import dataclass, field

import numpy as np

V_QWEN = 151936
V_262K = 262144


@dataclass
class Workload:
    name: str
    logits: np.ndarray            # [rows, vocab] float32
    vocab: int
    hist_ids: np.ndarray | None   # int32, concatenated
    hist_off: np.ndarray | None   # int64, rows + 1
    configs: list = field(default_factory=list)   # SampleConfig dicts
    uniforms: np.ndarray = None   # float64 [rows]

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    def history(self, r: int) -> np.ndarray:
        if self.hist_ids is None:
            return np.zeros(0, np.int32)
        return self.hist_ids[self.hist_off[r]:self.hist_off[r + 1]]

    def algorithmic_bytes(self) -> int:
        """sum over rows of 4*V + 4*H_eff + 4: H_eff = H with presence or
        frequency, min(H, 128) with only repetition, else 0."""
        total = 0
        for r, c in enumerate(self.configs):
            h = 0 if self.hist_off is None else int(self.hist_off[r + 1] - self.hist_off[r])
            pf = c.get("presencePenalty", 0) or c.get("frequencyPenalty", 0)
            rep = c.get("repetitionPenalty", 1.0) not in (None, 1.0)
            heff = h if pf else (min(h, 128) if rep else 0)
            total += 4 * self.vocab + 4 * heff + 4
        return total


def _normal_spiked(rng, rows, vocab, sigma=2.5, spikes=8, exact_spikes=False):
    x = rng.standard_normal((rows, vocab), dtype=np.float32)
    x *= np.float32(sigma)
    for r in range(rows):
        ids = rng.choice(vocab, size=min(spikes, vocab), replace=False)
        if exact_spikes:
            x[r, ids] = np.float32(12.0)
        else:
            x[r, ids] += np.float32(12.0)
    return x


def _zipf_ids(rng, n, vocab, s=1.1, perm=None):
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    p = ranks ** -s
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    r = np.minimum(r, vocab - 1)
    if perm is None:
        perm = rng.permutation(vocab)
    return perm[r].astype(np.int32)


def _pack(hists):
    off = np.zeros(len(hists) + 1, np.int64)
    for i, h in enumerate(hists):
        off[i + 1] = off[i] + len(h)
    ids = np.concatenate(hists).astype(np.int32) if hists else np.zeros(0, np.int32)
    return ids, off


def make(name: str, seed: int = 0, rows: int | None = None, vocab: int | None = None,
         greedy: bool = False, exact_spikes: bool = False) -> Workload:
    rng = np.random.default_rng([seed, sum(map(ord, name))])
    if name in ("single", "headline"):
        R = rows or (1 if name == "single" else 256)
        V = vocab or V_QWEN
        logits = _normal_spiked(rng, R, V, 2.5, 8, exact_spikes)
        hists = [rng.integers(0, V, 64).astype(np.int32) for _ in range(R)]
        cfg = dict(temperature=0.0 if greedy else 0.7, topK=40, topP=0.9,
                   repetitionPenalty=1.1)
        configs = [dict(cfg) for _ in range(R)]
    elif name == "batch64":
        R = rows or 64
        V = vocab or V_QWEN
        logits = _normal_spiked(rng, R, V, 2.5, 8, exact_spikes)
        hists = []
        for _ in range(R):
            pool = rng.integers(0, V, 48)
            hists.append(pool[rng.integers(0, pool.size, 256)].astype(np.int32))
        configs = [dict(temperature=0.8, topK=40, topP=0.95, repetitionPenalty=1.1)
                   for _ in range(R)]
    elif name == "perrow256":
        R = rows or 256
        V = vocab or V_QWEN
        logits = _normal_spiked(rng, R, V, 2.5, 8, exact_spikes)
        perm = rng.permutation(V)
        hists = [_zipf_ids(rng, 1024, V, 1.1, perm) for _ in range(R)]
        configs = []
        for _ in range(R):
            configs.append(dict(temperature=float(rng.uniform(0.3, 1.5)),
                                topK=int(rng.integers(1, min(1024, V) + 1)),
                                topP=float(rng.uniform(0.5, 0.99)),
                                presencePenalty=0.5, frequencyPenalty=0.3))
    elif name == "gumbel1024":
        R = rows or 1024
        V = vocab or V_QWEN
        u = rng.random((R, V))
        logits = np.empty((R, V), np.float32)

        def gumbel(a: int) -> None:   # row blocks in threads (numpy's log releases the GIL)
            logits[a:a + 64] = -np.log(-np.log(u[a:a + 64]))
        with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
            list(ex.map(gumbel, range(0, R, 64)))
        del u
        hists = None
        configs = [dict(temperature=1.0, topK=float("inf"), topP=0.98) for _ in range(R)]
    elif name == "v262k512":
        R = rows or 512
        V = vocab or V_262K
        logits = rng.standard_normal((R, V), dtype=np.float32) * np.float32(3.0)
        perm = rng.permutation(V)
        hists = [_zipf_ids(rng, 4096, V, 1.1, perm) for _ in range(R)]
        configs = [dict(temperature=0.9, topK=100, topP=0.9, repetitionPenalty=1.15,
                        presencePenalty=0.4, frequencyPenalty=0.2) for _ in range(R)]
    else:
        raise KeyError(f"unknown workload {name!r}")
    if hists is None:
        ids, off = None, None
    else:
        ids, off = _pack(hists)
    uniforms = rng.random(R)
    return Workload(name, np.ascontiguousarray(logits, np.float32), V, ids, off, configs,
                    uniforms)


NAMES = ("single", "batch64", "perrow256", "gumbel1024", "v262k512", "headline")


# ---- lm_head GEMV workloads ---------------------------------------------------

# GGML weight type ids (src/types.ts:4-15) and (weights, bytes) per block.
W_TYPES = {"f32": (0, 1, 4), "q4_0": (2, 32, 18), "q4_1": (3, 32, 20), "q4_k": (12, 256, 144),
           "q6_k": (14, 256, 210), "q1_0": (41, 128, 18), "pq2_0": (142, 128, 34),
           "ptq1_0": (143, 128, 28)}


@dataclass
class LmHead:
    """A synthetic lm_head: output.weight [vocab rows x hidden] in GGUF blocks
    of one format (random quants, binary16 scales near `scale`) and M hidden
    states x [M x hidden]."""
    wtype: int
    fmt: str
    vocab: int
    hidden: int
    weights: np.ndarray   # uint8 [vocab, row_bytes]
    x: np.ndarray         # float32 [M, hidden]

    def algorithmic_bytes(self) -> int:
        """The weights once, x once, the logits once."""
        return int(self.weights.nbytes + self.x.nbytes + 4 * self.x.shape[0] * self.vocab)


def make_lmhead(fmt: str = "q6_k", hidden: int = 2048, vocab: int = V_QWEN, m: int = 1,
                seed: int = 0, scale: float = 0.02) -> LmHead:
    wtype, bw, bb = W_TYPES[fmt]
    rng = np.random.default_rng([seed, hidden, wtype])
    x = rng.standard_normal((m, hidden)).astype(np.float32)
    if wtype == 0:
        w = (rng.standard_normal((vocab, hidden)) * scale).astype(np.float32).view(np.uint8)
        return LmHead(wtype, fmt, vocab, hidden, w, x)
    nb = hidden // bw
    raw = rng.integers(0, 256, (vocab, nb, bb), dtype=np.uint8)
    d = (rng.random((vocab, nb)) * 2 * scale).astype(np.float16).view(np.uint8).reshape(vocab, nb, 2)
    if wtype in (2, 3, 12):
        raw[:, :, 0:2] = d
    if wtype == 3:
        raw[:, :, 2:4] = (rng.standard_normal((vocab, nb)) * scale).astype(np.float16).view(
            np.uint8).reshape(vocab, nb, 2)
    if wtype == 12:
        raw[:, :, 2:4] = (rng.random((vocab, nb)) * scale).astype(np.float16).view(
            np.uint8).reshape(vocab, nb, 2)
    if wtype == 14:
        raw[:, :, 208:210] = d
    if wtype in (41, 142):
        raw[:, :, 0:2] = d
    if wtype == 143:
        raw[:, :, 26:28] = d
    return LmHead(wtype, fmt, vocab, hidden, raw.reshape(vocab, nb * bb), x)
