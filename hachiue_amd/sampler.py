"""Python host layer over the gfx950 sampler's C ABI (libhachiue_sampler.so).

Mirrors hachiue's ``sampleLogits(logits, vocab, history, config)``
(src/sampler.ts:12-118) and ``SampleConfig`` (src/sampler.ts:1-7): same
option names, the same `??` defaults (src/sampler.ts:18-22), the logits array
mutated in place by the penalties (src/sampler.ts:30) and the same
no-candidate return of 0 (src/sampler.ts:76).  The draw takes an injected
uniform in [0, 1) instead of ``Math.random()`` (src/sampler.ts:112).

There is no CPU fallback: every call runs the HIP kernels, and loading fails
loudly when the library or a GPU is missing.
"""
from __future__ import annotations

import ctypes
import math
import os
import random
from dataclasses import dataclass

import numpy as np

from . import hip

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libhachiue_sampler.so")

HS_OK = 0
ERROR_NAMES = {1: "HS_ERR_INVALID_ARGUMENT", 2: "HS_ERR_HIP", 3: "HS_ERR_OUT_OF_MEMORY",
               4: "HS_ERR_UNSUPPORTED"}

ROW_GREEDY, ROW_REPLAYED, ROW_TIES, ROW_SINGLE = 0x1, 0x2, 0x4, 0x8

# Every symbol include/hachiue_sampler.h declares.
EXPORTS = ("hs_abi_version", "hs_last_error", "hs_config_default", "hs_context_create",
           "hs_context_destroy", "hs_sample_logits", "hs_sample_logits_batch",
           "hs_sample_batch_device", "hs_sample_batch_device_ex",
           "hs_sample_batch_device_noalloc", "hs_argmax_device",
           "hs_argmax", "hs_gemv_device", "hs_gemv_device_ex", "hs_split_blocks",
           "hs_lm_head_sample_device", "hs_lm_head_sample_device_ex", "hs_decode_step_device",
           "hs_context_set_timing", "hs_context_kernel_times")


class SamplerError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(status, status)}: {message}")
        self.status = status


class WeightsC(ctypes.Structure):
    """hs_weights (include/hachiue_sampler.h): a weight tensor as the
    reference's GPU holds it (src/engine.ts:736-800)."""
    _fields_ = [("type", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
                ("hadamard", ctypes.c_int32), ("data", ctypes.c_void_p),
                ("scales16", ctypes.c_void_p), ("signs", ctypes.c_void_p)]


PLANAR_QUANT_BYTES = {41: 16, 142: 32, 143: 26}   # Q1_0, PQ2_0, PTQ1_0


def split_blocks(wtype: int, blocks) -> tuple[np.ndarray, np.ndarray]:
    """GGUF blocks of Q1_0 / PQ2_0 / PTQ1_0 -> (planar quants, binary16
    scales as uint8), through hs_split_blocks (src/engine.ts:80-175)."""
    qb = PLANAR_QUANT_BYTES[wtype]
    raw = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    n = raw.size // (qb + 2)
    if n * (qb + 2) != raw.size:
        raise ValueError("not a whole number of blocks")
    q = np.zeros(max(n * qb, 1), np.uint8)
    sc = np.zeros(max(n * 2, 1), np.uint8)
    P = ctypes.POINTER(ctypes.c_uint8)
    _check(lib().hs_split_blocks(int(wtype), raw.ctypes.data_as(P), n, q.ctypes.data_as(P),
                                 sc.ctypes.data_as(P)))
    return q[:n * qb], sc[:n * 2]


def weights(wtype: int, N: int, K: int, d_data: int, d_scales16: int | None = None,
            hadamard: bool = False, d_signs: int | None = None) -> WeightsC:
    return WeightsC(int(wtype), int(N), int(K), 1 if hadamard else 0, d_data, d_scales16 or None,
                    d_signs or None)


class SampleConfigC(ctypes.Structure):
    """hs_sample_config (include/hachiue_sampler.h)."""
    _fields_ = [("temperature", ctypes.c_double), ("top_k", ctypes.c_double),
                ("top_p", ctypes.c_double), ("min_p", ctypes.c_double),
                ("repetition_penalty", ctypes.c_double),
                ("presence_penalty", ctypes.c_double),
                ("frequency_penalty", ctypes.c_double)]


# SampleConfig option name -> hs_sample_config field, with the reference's
# defaults (src/sampler.ts:18-22) and 0 for the two extensions.
OPTIONS = {
    "temperature": ("temperature", 0.6),
    "topK": ("top_k", 20.0),
    "topP": ("top_p", 0.95),
    "minP": ("min_p", 0.0),
    "repetitionPenalty": ("repetition_penalty", 1.0),
    "presencePenalty": ("presence_penalty", 0.0),
    "frequencyPenalty": ("frequency_penalty", 0.0),
}
_FIELD_TO_OPTION = {f: o for o, (f, _) in OPTIONS.items()}


def resolve_config(config: dict | None) -> SampleConfigC:
    """`config.x ?? default` for every option: only a missing key or None takes
    the default.  Accepts the reference's camelCase names (and the snake_case
    field names); unknown keys are ignored, as extra GenerateOptions fields
    are (src/types.ts:187-197)."""
    c = SampleConfigC()
    for opt, (field, default) in OPTIONS.items():
        setattr(c, field, default)
    for key, val in (config or {}).items():
        opt = key if key in OPTIONS else _FIELD_TO_OPTION.get(key)
        if opt is None or val is None:
            continue
        setattr(c, OPTIONS[opt][0], float(val))
    return c


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    L = ctypes.CDLL(LIB_PATH)
    P, vp = ctypes.POINTER, ctypes.c_void_p
    i32, i64, dbl = ctypes.c_int32, ctypes.c_int64, ctypes.c_double
    L.hs_abi_version.restype = ctypes.c_int
    L.hs_last_error.restype = ctypes.c_char_p
    L.hs_config_default.argtypes = [P(SampleConfigC)]
    L.hs_config_default.restype = None
    L.hs_context_create.argtypes = [ctypes.c_int, P(vp)]
    L.hs_context_destroy.argtypes = [vp]
    L.hs_sample_logits.argtypes = [vp, P(ctypes.c_float), i32, P(i32), i64, P(SampleConfigC),
                                   dbl, P(i32)]
    L.hs_sample_logits_batch.argtypes = [vp, P(ctypes.c_float), i32, i64, i32, P(i32), P(i64),
                                         P(SampleConfigC), P(dbl), P(i32)]
    L.hs_sample_batch_device.argtypes = [vp, vp, i32, i64, i32, vp, vp, P(SampleConfigC), vp,
                                         vp, vp]
    L.hs_sample_batch_device_ex.argtypes = [vp, vp, i32, i64, i32, vp, vp, P(SampleConfigC),
                                            vp, vp, i32, vp, vp, vp, vp, vp, vp]
    L.hs_sample_batch_device_noalloc.argtypes = [vp, vp, i32, i64, i32, vp, vp,
                                                 P(SampleConfigC), vp, vp, vp]
    L.hs_argmax_device.argtypes = [vp, vp, i32, i64, i32, vp, vp]
    L.hs_argmax.argtypes = [vp, P(ctypes.c_float), i32, i64, i32, P(i32)]
    L.hs_gemv_device.argtypes = [vp, vp, i32, i64, i32, vp, i32, i32, vp, i64, vp]
    L.hs_lm_head_sample_device.argtypes = [vp, vp, i32, i64, i32, vp, i32, i32, vp, i64, vp, vp,
                                           P(SampleConfigC), vp, vp, vp]
    L.hs_gemv_device_ex.argtypes = [vp, vp, i32, i64, P(WeightsC), vp, i64, vp]
    L.hs_lm_head_sample_device_ex.argtypes = [vp, vp, i32, i64, P(WeightsC), vp, i64, vp, vp,
                                              P(SampleConfigC), vp, vp, vp]
    L.hs_split_blocks.argtypes = [i32, vp, i64, vp, vp]
    L.hs_decode_step_device.argtypes = [vp, vp, i32, i64, i32, vp, i64, vp, vp, vp, i32,
                                        P(SampleConfigC), vp, vp, vp]
    L.hs_context_set_timing.argtypes = [vp, ctypes.c_int]
    L.hs_context_kernel_times.argtypes = [vp, P(dbl), i32, P(i64)]
    return L


_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _check(status: int) -> None:
    if status != HS_OK:
        raise SamplerError(status, lib().hs_last_error().decode(errors="replace"))


def _f32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _histories(histories, rows):
    """(ids int32, offsets int64) from a list of id sequences, or a given
    (ids, offsets) pair.  Ids that are not integers in int32 range are
    stored as -1: in the reference they index nothing (src/sampler.ts:28)."""
    if histories is None:
        return None, None
    if isinstance(histories, tuple) and len(histories) == 2:
        ids = np.ascontiguousarray(histories[0], dtype=np.int32)
        off = np.ascontiguousarray(histories[1], dtype=np.int64)
        assert off.shape == (rows + 1,)
        return ids, off
    seqs = list(histories)
    assert len(seqs) == rows
    off = np.zeros(rows + 1, np.int64)
    parts = []
    for r, h in enumerate(seqs):
        a = _history_ids(h)
        parts.append(a)
        off[r + 1] = off[r] + a.size
    ids = np.concatenate(parts) if parts else np.zeros(0, np.int32)
    return np.ascontiguousarray(ids, dtype=np.int32), off


def _history_ids(h) -> np.ndarray:
    if isinstance(h, np.ndarray) and h.dtype.kind in "iu":
        a = h.astype(np.int64)
        return np.where((a >= -2**31) & (a < 2**31), a, -1).astype(np.int32)
    out = np.empty(len(h), np.int32)
    for i, x in enumerate(h):
        xf = float(x)
        out[i] = int(xf) if (math.isfinite(xf) and xf == int(xf) and -2**31 <= xf < 2**31) else -1
    return out


class Sampler:
    """One sampler context on one HIP device (not thread-safe)."""

    def __init__(self, device: int = 0):
        self._ctx = ctypes.c_void_p()
        _check(lib().hs_context_create(int(device), ctypes.byref(self._ctx)))
        self.device = device

    def close(self) -> None:
        if self._ctx.value:
            lib().hs_context_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    # ---- diagnostics ---------------------------------------------------------
    def set_timing(self, enable: bool) -> None:
        _check(lib().hs_context_set_timing(self._ctx, 1 if enable else 0))

    KERNELS = ("pen_kernel", "row_kernel", "chunk_kernel", "finalize_kernel", "large_kernel",
               "mid_kernel", "argmax_kernel", "gemv_kernel", "large_fast_kernel",
               "large_replay_kernel", "large_replay_dev_kernel")

    def kernel_times(self):
        """({kernel: total device ms}, calls) since the last query."""
        ms = (ctypes.c_double * len(self.KERNELS))()
        calls = ctypes.c_int64()
        _check(lib().hs_context_kernel_times(self._ctx, ms, len(self.KERNELS), ctypes.byref(calls)))
        return {k: float(ms[i]) for i, k in enumerate(self.KERNELS)}, int(calls.value)

    # ---- drop-in: one host row -------------------------------------------
    def sample_logits(self, logits: np.ndarray, vocab: int, history=(), config: dict | None = None,
                      uniform: float | None = None) -> int:
        """sampleLogits(logits, vocab, history, config) on the GPU.  `logits`
        (float32, contiguous, length >= vocab) receives the penalised values
        in place.  Without `uniform`, ``random.random()`` stands in for
        Math.random() and is drawn only when the reference would draw
        (draw_rule)."""
        if not (isinstance(logits, np.ndarray) and logits.dtype == np.float32
                and logits.flags.c_contiguous):
            raise TypeError("logits must be a contiguous float32 numpy array")
        vocab = int(vocab)
        cfg = resolve_config(config)
        if vocab > logits.size:
            raise ValueError("vocab exceeds the logits length")
        ids = _history_ids(list(history) if not isinstance(history, np.ndarray) else history)
        rule = DRAW if uniform is not None else draw_rule(cfg, vocab, logits, ids)
        if rule != DRAW_UNKNOWN:
            if uniform is None:
                uniform = random.random() if rule == DRAW else 0.0
            return self._sample_row(logits, vocab, ids, cfg, float(uniform))
        # a penalty decides whether two candidates remain: penalise and sample
        # without a draw, then draw on the penalised row only if it has them
        tok = self._sample_row(logits, vocab, ids, cfg, 0.0)
        if _two_candidates(logits, vocab):
            tok = self._sample_row(logits, vocab, np.zeros(0, np.int32), _without_penalties(cfg),
                                   random.random())
        return tok

    def _sample_row(self, logits, vocab, ids, cfg, uniform: float) -> int:
        tok = ctypes.c_int32()
        _check(lib().hs_sample_logits(self._ctx, _f32p(logits), vocab,
                                      ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                      int(ids.size), ctypes.byref(cfg), uniform,
                                      ctypes.byref(tok)))
        return int(tok.value)

    # ---- batch over host buffers ------------------------------------------
    def sample_logits_batch(self, logits: np.ndarray, vocab: int, histories=None, configs=None,
                            uniforms=None) -> np.ndarray:
        """Rows of a [rows, stride] float32 array, each with its own history,
        config and uniform.  Penalised values are written back in place."""
        if not (isinstance(logits, np.ndarray) and logits.dtype == np.float32
                and logits.ndim == 2 and logits.flags.c_contiguous):
            raise TypeError("logits must be a contiguous 2-D float32 numpy array")
        rows, stride = logits.shape
        cfgs = _configs(configs, rows)
        ids, off = _histories(histories, rows)
        second = False
        if uniforms is None:
            # random.random() once for each row that draws, in row order
            rules = [draw_rule(cfgs[r], int(vocab), logits[r],
                               ids[off[r]:off[r + 1]] if ids is not None else None)
                     for r in range(rows)] if vocab > 0 else [NO_DRAW] * rows
            second = DRAW_UNKNOWN in rules
            u = np.zeros(rows) if second else np.array(
                [random.random() if x == DRAW else 0.0 for x in rules])
        else:
            u = np.ascontiguousarray(uniforms, dtype=np.float64)
        tok = self._batch(logits, vocab, ids, off, cfgs, u)
        if not second:
            return tok
        # pass 1 applied the penalties without drawing; the draws follow the
        # penalised rows
        u = np.array([random.random() if rules[r] == DRAW or (
            rules[r] == DRAW_UNKNOWN and _two_candidates(logits[r], int(vocab))) else 0.0
            for r in range(rows)])
        plain = (SampleConfigC * rows)(*[_without_penalties(c) for c in cfgs])
        return self._batch(logits, vocab, None, None, plain, u)

    def _batch(self, logits, vocab, ids, off, cfgs, u) -> np.ndarray:
        rows, stride = logits.shape
        tok = np.zeros(rows, np.int32)
        P = ctypes.POINTER
        _check(lib().hs_sample_logits_batch(
            self._ctx, _f32p(logits), rows, stride, int(vocab),
            ids.ctypes.data_as(P(ctypes.c_int32)) if ids is not None else None,
            off.ctypes.data_as(P(ctypes.c_int64)) if off is not None else None,
            cfgs, u.ctypes.data_as(P(ctypes.c_double)), tok.ctypes.data_as(P(ctypes.c_int32))))
        return tok

    # ---- the engine's GPU greedy route -----------------------------------------
    def argmax(self, logits: np.ndarray, vocab: int | None = None) -> np.ndarray:
        """The WGSL argmax of src/kernels.ts:1613-1654 (the engine's greedy
        route without a repetition penalty, src/engine.ts:1600-1601) over the
        rows of a 1-D or 2-D float32 array; logits are read only."""
        if not (isinstance(logits, np.ndarray) and logits.dtype == np.float32
                and logits.flags.c_contiguous):
            raise TypeError("logits must be a contiguous float32 numpy array")
        x = logits.reshape(1, -1) if logits.ndim == 1 else logits
        rows, stride = x.shape
        vocab = stride if vocab is None else int(vocab)
        if vocab > stride:
            raise ValueError("vocab exceeds the row length")
        tok = np.zeros(rows, np.int32)
        _check(lib().hs_argmax(self._ctx, _f32p(x), rows, stride, vocab,
                               tok.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))))
        return tok

    def argmax_device(self, d_logits: int, rows: int, row_stride: int, vocab: int,
                      d_tokens: int, stream=None) -> None:
        """Enqueue the greedy-route argmax on device buffers (addresses as ints)."""
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_argmax_device(self._ctx, vp(d_logits), int(rows), int(row_stride),
                                      int(vocab), vp(d_tokens), st))

    # ---- lm_head GEMV -----------------------------------------------------------
    def gemv_device(self, d_x: int, M: int, ldx: int, K: int, d_w: int, w_type: int, N: int,
                    d_y: int, ldy: int, stream=None) -> None:
        """y = x W^T on device buffers (addresses as ints); W in GGML blocks."""
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_gemv_device(self._ctx, vp(d_x), int(M), int(ldx), int(K), vp(d_w),
                                    int(w_type), int(N), vp(d_y), int(ldy), st))

    def gemv_device_ex(self, d_x: int, M: int, ldx: int, w: WeightsC, d_y: int, ldy: int,
                       stream=None) -> None:
        """y = x W^T for any hs_weights (planar Q1_0 / PQ2_0 / PTQ1_0, and
        Hadamard-folded weights)."""
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_gemv_device_ex(self._ctx, vp(d_x), int(M), int(ldx), ctypes.byref(w),
                                       vp(d_y), int(ldy), st))

    def lm_head_sample_device_ex(self, d_x: int, M: int, ldx: int, w: WeightsC, d_logits: int,
                                 ldl: int, d_hist_ids, d_hist_off, configs, d_uniforms: int,
                                 d_tokens: int, stream=None) -> None:
        """gemv_device_ex into d_logits, then sampling of its M rows."""
        cfgs = configs if isinstance(configs, ctypes.Array) else _configs(configs, M)
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_lm_head_sample_device_ex(
            self._ctx, vp(d_x), int(M), int(ldx), ctypes.byref(w), vp(d_logits), int(ldl),
            vp(d_hist_ids or 0), vp(d_hist_off or 0), cfgs, vp(d_uniforms), vp(d_tokens), st))

    def lm_head_sample_device(self, d_x: int, M: int, ldx: int, K: int, d_w: int, w_type: int,
                              N: int, d_logits: int, ldl: int, d_hist_ids, d_hist_off, configs,
                              d_uniforms: int, d_tokens: int, stream=None) -> None:
        """The lm_head GEMV into d_logits, then sampling of its M rows."""
        cfgs = configs if isinstance(configs, ctypes.Array) else _configs(configs, M)
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_lm_head_sample_device(
            self._ctx, vp(d_x), int(M), int(ldx), int(K), vp(d_w), int(w_type), int(N),
            vp(d_logits), int(ldl), vp(d_hist_ids or 0), vp(d_hist_off or 0), cfgs,
            vp(d_uniforms), vp(d_tokens), st))

    def decode_step_device(self, d_logits: int, rows: int, row_stride: int, vocab: int,
                           d_ring: int, ring_cap: int, d_len: int, d_done: int,
                           d_stop_ids: int | None, n_stop: int, configs, d_uniforms: int,
                           d_tokens: int, stream=None) -> None:
        """One decode step (src/engine.ts:1626-1644) with the histories in
        device rings: draw, stop check, history append, no synchronisation."""
        cfgs = configs if isinstance(configs, ctypes.Array) else _configs(configs, rows)
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_decode_step_device(
            self._ctx, vp(d_logits), int(rows), int(row_stride), int(vocab), vp(d_ring),
            int(ring_cap), vp(d_len), vp(d_done), vp(d_stop_ids or 0), int(n_stop), cfgs,
            vp(d_uniforms), vp(d_tokens), st))

    # ---- device-resident batch ----------------------------------------------
    def sample_device(self, d_logits: int, rows: int, row_stride: int, vocab: int,
                      d_hist_ids: int | None, d_hist_off: int | None, configs,
                      d_uniforms: int, d_tokens: int, stream=None,
                      cand_stride: int = 0, d_cand_ids: int | None = None,
                      d_cand_probs: int | None = None, d_cand_count: int | None = None,
                      d_cutoff: int | None = None, d_row_flags: int | None = None) -> None:
        """Enqueue one sampling step on device buffers (addresses as ints)."""
        cfgs = configs if isinstance(configs, ctypes.Array) else _configs(configs, rows)
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_sample_batch_device_ex(
            self._ctx, vp(d_logits), int(rows), int(row_stride), int(vocab), vp(d_hist_ids or 0),
            vp(d_hist_off or 0), cfgs, vp(d_uniforms), vp(d_tokens), int(cand_stride),
            vp(d_cand_ids or 0), vp(d_cand_probs or 0), vp(d_cand_count or 0), vp(d_cutoff or 0),
            vp(d_row_flags or 0), st))


    def sample_device_noalloc(self, d_logits: int, rows: int, row_stride: int, vocab: int,
                              d_hist_ids: int | None, d_hist_off: int | None, configs,
                              d_uniforms: int, d_tokens: int, stream=None) -> None:
        """sample_device through hs_sample_batch_device_noalloc: the same
        step with the GPU's static scratch array as the workspace."""
        cfgs = configs if isinstance(configs, ctypes.Array) else _configs(configs, rows)
        vp = ctypes.c_void_p
        st = stream.handle if isinstance(stream, hip.Stream) else stream
        _check(lib().hs_sample_batch_device_noalloc(
            self._ctx, vp(d_logits), int(rows), int(row_stride), int(vocab), vp(d_hist_ids or 0),
            vp(d_hist_off or 0), cfgs, vp(d_uniforms), vp(d_tokens), st))


def _configs(configs, rows: int):
    if configs is None or isinstance(configs, dict):
        one = resolve_config(configs)
        return (SampleConfigC * rows)(*([one] * rows))
    configs = list(configs)
    if len(configs) != rows:
        raise ValueError("one config per row is required")
    return (SampleConfigC * rows)(*[resolve_config(c) for c in configs])


def greedy_route(options: dict | None) -> bool:
    """src/engine.ts:1600-1601: the engine decodes with the GPU argmax instead
    of sampleLogits when (temperature ?? 0.6) <= 0 and no repetition penalty
    other than 1.0 is given."""
    o = options or {}
    t = o.get("temperature")
    rp = o.get("repetitionPenalty")
    return (0.6 if t is None else t) <= 0 and (rp is None or rp == 1.0)


def make_configs(configs, rows: int):
    """ctypes array of hs_sample_config for `rows` rows (dict = shared)."""
    return _configs(configs, rows)


DRAW, NO_DRAW, DRAW_UNKNOWN = 1, 0, -1


def draw_rule(cfg: SampleConfigC, vocab: int, row: np.ndarray, hist: np.ndarray | None) -> int:
    """Whether sampleLogits calls Math.random() for this row
    (src/sampler.ts:36, :49-50, :76-77, :112): once iff !(temperature <= 0)
    (a NaN temperature draws) and order.length >= 2, where order.length is
    min(k, the number of penalised logits > -Infinity).  Penalties touch only
    history ids, so two logits > -Infinity at ids outside the history settle
    it before the call.  Returns DRAW, NO_DRAW, or DRAW_UNKNOWN when only the
    penalised row can tell."""
    if cfg.temperature <= 0:
        return NO_DRAW
    t = cfg.top_k if cfg.top_k > 0 else 64.0
    if math.floor(max(1.0, min(t, float(vocab)))) < 2:
        return NO_DRAW
    rep = cfg.repetition_penalty != 1.0
    pf = cfg.presence_penalty != 0.0 or cfg.frequency_penalty != 0.0
    h = np.zeros(0, np.int32) if hist is None else np.asarray(hist)
    window = h if pf else h[-128:]
    touched = (rep or pf) and window.size > 0
    cand = row[:vocab] > -np.inf
    if touched:
        ids = window[(window >= 0) & (window < vocab)]
        cand[ids] = False
    if int(np.count_nonzero(cand)) >= 2:
        return DRAW
    return DRAW_UNKNOWN if touched else NO_DRAW


def _two_candidates(row: np.ndarray, vocab: int) -> bool:
    return int(np.count_nonzero(row[:vocab] > -np.inf)) >= 2


def _without_penalties(cfg: SampleConfigC) -> SampleConfigC:
    c = SampleConfigC()
    ctypes.memmove(ctypes.byref(c), ctypes.byref(cfg), ctypes.sizeof(c))
    c.repetition_penalty, c.presence_penalty, c.frequency_penalty = 1.0, 0.0, 0.0
    return c


@dataclass
class DeviceOutputs:
    tokens: hip.DeviceArray
    cand_ids: hip.DeviceArray | None
    cand_probs: hip.DeviceArray | None
    cand_count: hip.DeviceArray | None
    cutoff: hip.DeviceArray | None
    row_flags: hip.DeviceArray | None


_default: Sampler | None = None


def default_sampler() -> Sampler:
    global _default
    if _default is None:
        _default = Sampler(0)
    return _default


def sample_logits(logits: np.ndarray, vocab: int, history=(), config: dict | None = None,
                  uniform: float | None = None) -> int:
    """Module-level drop-in for sampleLogits on the default GPU context."""
    return default_sampler().sample_logits(logits, vocab, history, config, uniform)
