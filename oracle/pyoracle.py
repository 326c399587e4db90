"""ctypes binding of the CPU oracle (liborc_sampler.so).

TEST INFRASTRUCTURE ONLY: the oracle is the checker the HIP sampler is
compared against.  Only tests, the smoke check and the benchmark's CPU
baseline import this module; the product package never does.

The oracle restates hachiue's ``sampleLogits`` (src/sampler.ts:12-118); see
``sampler_oracle.c`` for the line-by-line correspondence.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liborc_sampler.so")

LITERAL = 0  # the reference's O(V*k) replace-min rescan, verbatim
HEAP = 1     # identical slot semantics, O(V + R log k)


class OrcConfig(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_double),
        ("top_k", ctypes.c_double),
        ("top_p", ctypes.c_double),
        ("min_p", ctypes.c_double),
        ("repetition_penalty", ctypes.c_double),
        ("presence_penalty", ctypes.c_double),
        ("frequency_penalty", ctypes.c_double),
    ]


class OrcResult(ctypes.Structure):
    _fields_ = [
        ("token", ctypes.c_int32),
        ("path", ctypes.c_int32),
        ("k", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("cutoff", ctypes.c_int32),
        ("draw_index", ctypes.c_int32),
        ("sum_prob", ctypes.c_double),
        ("kept_sum", ctypes.c_double),
        ("draw_margin", ctypes.c_double),
        ("topp_margin", ctypes.c_double),
    ]


# src/sampler.ts:18-22 defaults
DEFAULTS = dict(temperature=0.6, top_k=20.0, top_p=0.95, min_p=0.0,
                repetition_penalty=1.0, presence_penalty=0.0,
                frequency_penalty=0.0)

_CFG_KEYS = {"temperature": "temperature", "topK": "top_k", "topP": "top_p",
             "minP": "min_p", "repetitionPenalty": "repetition_penalty",
             "presencePenalty": "presence_penalty",
             "frequencyPenalty": "frequency_penalty"}


def resolve_config(cfg: dict | None) -> dict:
    """Apply the reference's `??` defaults: only a missing key or None takes
    the default (src/sampler.ts:18-22).  Accepts camelCase or snake_case."""
    out = dict(DEFAULTS)
    for key, val in (cfg or {}).items():
        name = _CFG_KEYS.get(key, key)
        if name not in out:
            raise KeyError(f"unknown sampler option {key!r}")
        if val is not None:
            out[name] = float(val)
    return out


def make_config(cfg: dict | None) -> OrcConfig:
    r = resolve_config(cfg)
    return OrcConfig(**r)


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER
        L.orc_resolve_k.restype = ctypes.c_int64
        L.orc_resolve_k.argtypes = [ctypes.c_double, ctypes.c_int64]
        L.orc_apply_penalties.restype = None
        L.orc_apply_penalties.argtypes = [P(ctypes.c_float), ctypes.c_int64,
                                          P(ctypes.c_int32), ctypes.c_int64,
                                          P(OrcConfig)]
        L.orc_sample_row.restype = ctypes.c_int
        L.orc_sample_row.argtypes = [P(ctypes.c_float), ctypes.c_int64,
                                     P(ctypes.c_int32), ctypes.c_int64,
                                     P(OrcConfig), ctypes.c_double, ctypes.c_int,
                                     P(OrcResult), P(ctypes.c_int32),
                                     P(ctypes.c_float), P(ctypes.c_float),
                                     ctypes.c_int64]
        L.orc_sample_batch.restype = ctypes.c_int
        L.orc_sample_batch.argtypes = [P(ctypes.c_float), ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_int64,
                                       P(ctypes.c_int32), P(ctypes.c_int64),
                                       P(OrcConfig), P(ctypes.c_double),
                                       ctypes.c_int, P(OrcResult),
                                       P(ctypes.c_int32), P(ctypes.c_float),
                                       P(ctypes.c_float), ctypes.c_int64]
        L.orc_block_weights.restype = ctypes.c_int
        L.orc_block_weights.argtypes = [ctypes.c_int]
        L.orc_block_bytes.restype = ctypes.c_int
        L.orc_block_bytes.argtypes = [ctypes.c_int]
        L.orc_fp16.restype = ctypes.c_float
        L.orc_fp16.argtypes = [ctypes.c_uint16]
        L.orc_dequant_row.restype = ctypes.c_int
        L.orc_dequant_row.argtypes = [ctypes.c_int, P(ctypes.c_uint8), ctypes.c_int64,
                                      P(ctypes.c_float)]
        L.orc_gemv_exact.restype = ctypes.c_int
        L.orc_gemv_exact.argtypes = [ctypes.c_int, P(ctypes.c_float), ctypes.c_int64,
                                     ctypes.c_int64, P(ctypes.c_uint8), ctypes.c_int64,
                                     P(ctypes.c_double), P(ctypes.c_double)]
        L.orc_gemv_ref.restype = ctypes.c_int
        L.orc_gemv_ref.argtypes = [ctypes.c_int, P(ctypes.c_float), ctypes.c_int64,
                                   ctypes.c_int64, P(ctypes.c_uint8), ctypes.c_int64,
                                   P(ctypes.c_float)]
        L.orc_hadamard512.restype = ctypes.c_int
        L.orc_hadamard512.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64,
                                      P(ctypes.c_float)]
        L.orc_wgsl_argmax.restype = None
        L.orc_wgsl_argmax.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_int64, P(ctypes.c_int32)]
        L.orc_wasm_greedy.restype = None
        L.orc_wasm_greedy.argtypes = [P(ctypes.c_float), ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_int64, P(ctypes.c_int32)]
        L.orc_topk_slots.restype = ctypes.c_int
        L.orc_topk_slots.argtypes = [P(ctypes.c_float), ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int,
                                     P(ctypes.c_int32), P(ctypes.c_float)]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None, ct):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ct))


@dataclass
class RowResult:
    token: int
    path: int
    k: int
    n: int
    cutoff: int
    draw_index: int
    sum_prob: float
    kept_sum: float
    draw_margin: float
    topp_margin: float
    cand_ids: np.ndarray
    cand_vals: np.ndarray
    cand_probs: np.ndarray


def resolve_k(top_k: float, vocab: int) -> int:
    return int(lib().orc_resolve_k(float(top_k), int(vocab)))


def apply_penalties(logits: np.ndarray, vocab: int, history, cfg: dict | None) -> None:
    assert logits.dtype == np.float32 and logits.flags.c_contiguous
    h = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
    c = make_config(cfg)
    lib().orc_apply_penalties(_ptr(logits, ctypes.c_float), int(vocab),
                              _ptr(h, ctypes.c_int32), int(h.size), ctypes.byref(c))


def sample_row(logits: np.ndarray, vocab: int, history, cfg: dict | None,
               u: float, method: int = HEAP, cap: int | None = None) -> RowResult:
    """sampleLogits on one row; `logits` (float32, contiguous) is mutated in
    place like the reference's Float32Array."""
    assert logits.dtype == np.float32 and logits.flags.c_contiguous
    h = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
    c = make_config(cfg)
    if cap is None:
        cap = resolve_k(c.top_k, vocab)
    ids = np.full(cap, -1, np.int32)
    vals = np.zeros(cap, np.float32)
    probs = np.zeros(cap, np.float32)
    res = OrcResult()
    rc = lib().orc_sample_row(_ptr(logits, ctypes.c_float), int(vocab),
                              _ptr(h, ctypes.c_int32), int(h.size),
                              ctypes.byref(c), float(u), int(method),
                              ctypes.byref(res), _ptr(ids, ctypes.c_int32),
                              _ptr(vals, ctypes.c_float),
                              _ptr(probs, ctypes.c_float), int(cap))
    if rc:
        raise MemoryError("oracle allocation failed")
    n = min(res.n, cap)
    return RowResult(res.token, res.path, res.k, res.n, res.cutoff,
                     res.draw_index, res.sum_prob, res.kept_sum,
                     res.draw_margin, res.topp_margin, ids[:n].copy(),
                     vals[:n].copy(), probs[:n].copy())


@dataclass
class BatchResult:
    token: np.ndarray
    path: np.ndarray
    n: np.ndarray
    cutoff: np.ndarray
    draw_index: np.ndarray
    draw_margin: np.ndarray
    topp_margin: np.ndarray
    cand_ids: np.ndarray | None
    cand_vals: np.ndarray | None
    cand_probs: np.ndarray | None


def sample_batch(logits: np.ndarray, vocab: int, hist_ids: np.ndarray | None,
                 hist_off: np.ndarray | None, cfgs: list[dict] | dict,
                 u: np.ndarray, method: int = HEAP, cap: int = 0,
                 threads: int | None = None) -> BatchResult:
    """Row-by-row oracle over a [rows, stride] float32 batch (mutated in place).
    Large batches run in blocks of rows on `threads` threads (the C call
    releases the GIL); the rows are independent, so the result is the same."""
    assert logits.dtype == np.float32 and logits.ndim == 2 and logits.flags.c_contiguous
    rows, stride = logits.shape
    if isinstance(cfgs, dict) or cfgs is None:
        cfgs = [cfgs] * rows
    threads = min(16, os.cpu_count() or 1) if threads is None else threads
    if threads > 1 and rows >= 32:
        return _sample_blocks(logits, vocab, hist_ids, hist_off, cfgs, u, method, cap, threads)
    carr = (OrcConfig * rows)(*[make_config(c) for c in cfgs])
    u = np.ascontiguousarray(u, dtype=np.float64)
    res = (OrcResult * rows)()
    ids = np.full((rows, max(cap, 1)), -1, np.int32) if cap else None
    vals = np.zeros((rows, max(cap, 1)), np.float32) if cap else None
    probs = np.zeros((rows, max(cap, 1)), np.float32) if cap else None
    if hist_ids is not None:
        hist_ids = np.ascontiguousarray(hist_ids, dtype=np.int32)
        hist_off = np.ascontiguousarray(hist_off, dtype=np.int64)
    rc = lib().orc_sample_batch(_ptr(logits, ctypes.c_float), rows, stride,
                                int(vocab), _ptr(hist_ids, ctypes.c_int32),
                                _ptr(hist_off, ctypes.c_int64), carr,
                                _ptr(u, ctypes.c_double), int(method), res,
                                _ptr(ids, ctypes.c_int32), _ptr(vals, ctypes.c_float),
                                _ptr(probs, ctypes.c_float), int(cap))
    if rc:
        raise MemoryError("oracle allocation failed")
    g = lambda f: np.array([getattr(r, f) for r in res])  # noqa: E731
    return BatchResult(g("token").astype(np.int32), g("path"), g("n"), g("cutoff"),
                       g("draw_index"), g("draw_margin"), g("topp_margin"),
                       ids, vals, probs)


def _sample_blocks(logits, vocab, hist_ids, hist_off, cfgs, u, method, cap, threads):
    from concurrent.futures import ThreadPoolExecutor
    rows = logits.shape[0]
    u = np.ascontiguousarray(u, dtype=np.float64)
    step = max(8, -(-rows // (4 * threads)))
    blocks = [(a, min(rows, a + step)) for a in range(0, rows, step)]

    def one(ab):
        a, b = ab
        ids = off = None
        if hist_ids is not None:
            o = np.asarray(hist_off, np.int64)
            ids = np.ascontiguousarray(hist_ids[o[a]:o[b]], dtype=np.int32)
            off = o[a:b + 1] - o[a]
        return sample_batch(logits[a:b], vocab, ids, off, cfgs[a:b], u[a:b], method, cap,
                            threads=1)
    with ThreadPoolExecutor(max_workers=threads) as ex:
        parts = list(ex.map(one, blocks))
    cat = lambda f: np.concatenate([getattr(p, f) for p in parts])  # noqa: E731
    return BatchResult(cat("token"), cat("path"), cat("n"), cat("cutoff"), cat("draw_index"),
                       cat("draw_margin"), cat("topp_margin"),
                       cat("cand_ids") if cap else None, cat("cand_vals") if cap else None,
                       cat("cand_probs") if cap else None)


def topk_slots(logits: np.ndarray, vocab: int, k: int, method: int = LITERAL):
    ids = np.full(k, -1, np.int32)
    vals = np.full(k, -np.inf, np.float32)
    rc = lib().orc_topk_slots(_ptr(np.ascontiguousarray(logits, np.float32), ctypes.c_float),
                              int(vocab), int(k), int(method),
                              _ptr(ids, ctypes.c_int32), _ptr(vals, ctypes.c_float))
    if rc:
        raise MemoryError("oracle allocation failed")
    return ids, vals


def wgsl_argmax(logits: np.ndarray, vocab: int, rows: int | None = None,
                stride: int | None = None) -> np.ndarray:
    """The engine's GPU greedy route (src/engine.ts:1600-1601): the WGSL
    argmax of src/kernels.ts:1613-1654, one id per row."""
    x = np.ascontiguousarray(logits, np.float32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    rows = x.shape[0] if rows is None else rows
    stride = x.shape[1] if stride is None else stride
    out = np.zeros(rows, np.int32)
    lib().orc_wgsl_argmax(_ptr(x, ctypes.c_float), rows, stride, vocab,
                          _ptr(out, ctypes.c_int32))
    return out


def wasm_greedy(logits: np.ndarray, vocab: int, rows: int | None = None,
                stride: int | None = None) -> np.ndarray:
    """The Wasm backend's greedy route (src/wasm-backend.ts:1204-1215), one
    id per row: the first id of the largest logit above -1e30."""
    x = np.ascontiguousarray(logits, np.float32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    rows = x.shape[0] if rows is None else rows
    stride = x.shape[1] if stride is None else stride
    out = np.zeros(rows, np.int32)
    lib().orc_wasm_greedy(_ptr(x, ctypes.c_float), rows, stride, vocab,
                          _ptr(out, ctypes.c_int32))
    return out


# ---- lm_head GEMV (oracle/lmhead_oracle.h) ----------------------------------
W_F32, W_Q4_0, W_Q4_1, W_Q4_K, W_Q6_K = 0, 2, 3, 12, 14
W_Q1_0, W_PQ2_0, W_PTQ1_0 = 41, 142, 143


def block_spec(wtype: int) -> tuple[int, int]:
    """(weights per block, bytes per block) of a GGML type (src/gguf.ts getBlockSpec)."""
    return lib().orc_block_weights(wtype), lib().orc_block_bytes(wtype)


def fp16(h: int) -> float:
    return float(lib().orc_fp16(h))


def dequant_row(wtype: int, row: np.ndarray, K: int) -> np.ndarray:
    """One row of W dequantised as src/gguf.ts:149-230 does (binary32)."""
    row = np.ascontiguousarray(row, np.uint8)
    out = np.zeros(K, np.float32)
    if lib().orc_dequant_row(wtype, _ptr(row, ctypes.c_uint8), K, _ptr(out, ctypes.c_float)):
        raise ValueError("bad type or K")
    return out


def gemv_exact(wtype: int, x: np.ndarray, w: np.ndarray, N: int):
    """(y, mag): y = x W^T in binary64 from the exact weights, mag = sum |x w|."""
    x = np.ascontiguousarray(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    w = np.ascontiguousarray(w, np.uint8)
    y = np.zeros((M, N), np.float64)
    mag = np.zeros((M, N), np.float64)
    if lib().orc_gemv_exact(wtype, _ptr(x2, ctypes.c_float), M, K, _ptr(w, ctypes.c_uint8), N,
                            _ptr(y, ctypes.c_double), _ptr(mag, ctypes.c_double)):
        raise ValueError("bad type or K")
    return y, mag


def hadamard512(x: np.ndarray, signs: np.ndarray | None = None) -> np.ndarray:
    """The 512-wide rotation of a hadamard-folded weight's input
    (src/kernels.ts:177-227, mode 0): a rotated copy of x [M x K]."""
    y = np.array(x, np.float32, copy=True, order="C")
    y2 = y.reshape(-1, y.shape[-1])
    s = None if signs is None else np.ascontiguousarray(signs, np.float32)
    if lib().orc_hadamard512(_ptr(y2, ctypes.c_float), y2.shape[0], y2.shape[1],
                             _ptr(s, ctypes.c_float)):
        raise ValueError("width must be a multiple of 512")
    return y


def gemv_ref(wtype: int, x: np.ndarray, w: np.ndarray, N: int) -> np.ndarray:
    """The reference's binary32 GEMV result in its own summation order."""
    x = np.ascontiguousarray(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    w = np.ascontiguousarray(w, np.uint8)
    y = np.zeros((M, N), np.float32)
    if lib().orc_gemv_ref(wtype, _ptr(x2, ctypes.c_float), M, K, _ptr(w, ctypes.c_uint8), N,
                          _ptr(y, ctypes.c_float)):
        raise ValueError("bad type or K")
    return y


# ---- the decode loop (src/engine.ts:1626-1644) ------------------------------

class DecodeResult:
    def __init__(self, tokens, histories, done, steps):
        self.tokens = tokens          # [steps][rows] int32, -1 once a row is done
        self.histories = histories    # per row: prompt + appended ids
        self.done = done              # per row: a stop id was drawn
        self.steps = steps            # per step: the BatchResult of its draw


def decode_loop(step_logits, vocab: int, prompts, stop_ids, cfgs, uniforms,
                ring_cap: int | None = None) -> DecodeResult:
    """src/engine.ts:1626-1644 for independent rows: at each step every row
    draws from that step's logits ([rows, stride] float32, mutated like the
    reference's) with its token history (src/sampler.ts through sample_batch);
    a drawn stop id ends the row before it joins the history (:1628), any
    other id is pushed to the history (:1638), and a row once done reports
    -1.  With ring_cap, a draw sees only the last ring_cap history ids (what a
    device ring of that capacity holds)."""
    rows = len(prompts)
    hist = [list(int(t) for t in p) for p in prompts]
    done = [False] * rows
    stop = set(int(t) for t in stop_ids)
    tokens, results = [], []
    for s, logits in enumerate(step_logits):
        seen = [h[-ring_cap:] if ring_cap else h for h in hist]
        off = np.zeros(rows + 1, np.int64)
        for r, h in enumerate(seen):
            off[r + 1] = off[r] + len(h)
        ids = np.array([t for h in seen for t in h], np.int32)
        res = sample_batch(logits, vocab, ids, off, cfgs, uniforms[s])
        row_tok = []
        for r in range(rows):
            if done[r]:
                row_tok.append(-1)
                continue
            t = int(res.token[r])
            row_tok.append(t)
            if t in stop:
                done[r] = True
            else:
                hist[r].append(t)
        tokens.append(row_tok)
        results.append(res)
    return DecodeResult(np.array(tokens, np.int32).reshape(len(tokens), rows), hist, done,
                        results)
