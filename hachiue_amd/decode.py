"""Device-resident decode state: the engine's token history and stop check
(src/engine.ts:1591-1644) kept on the GPU between steps.

The reference keeps `tokenHistory` as a host array, reads every step's logits
back to the host (src/engine.ts:1526-1531) and checks `stopSet` there.  A
DecodeState keeps, per sequence row, a ring of the last `ring_cap` history
ids, the count of ids appended, and a done flag in device memory; each
`step` draws the next token of every row from device logits, applies the
stop check and appends the token, all enqueued on one stream through
hs_decode_step_device.  The host reads tokens and flags only when it wants
them.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import hip
from .sampler import Sampler, _configs


class DecodeState:
    """Rows of decode state: rings [rows][ring_cap] int32, len [rows] int64,
    done [rows] int32, and the stop set (src/engine.ts:1592-1598: the EOS id
    plus options.stopTokens and the model's end-of-message ids)."""

    def __init__(self, sampler: Sampler, prompts, stop_ids=(), ring_cap: int = 4096):
        if ring_cap < 128:
            raise ValueError("ring_cap must be >= 128 (the repetition-penalty window)")
        self.sampler = sampler
        self.rows = len(prompts)
        self.ring_cap = int(ring_cap)
        ring = np.zeros((self.rows, self.ring_cap), np.int32)
        lens = np.zeros(self.rows, np.int64)
        for r, p in enumerate(prompts):
            ids = np.asarray(p, np.int64).reshape(-1)
            lens[r] = ids.size
            keep = ids[-self.ring_cap:] if ids.size else ids
            pos = (np.arange(ids.size - keep.size, ids.size)) % self.ring_cap
            ring[r, pos] = keep.astype(np.int32)
        stop = np.unique(np.asarray(list(stop_ids), np.int64)).astype(np.int32)
        self.n_stop = int(stop.size)
        self.ring = hip.DeviceArray.from_numpy(ring)
        self.len = hip.DeviceArray.from_numpy(lens)
        self.done = hip.DeviceArray.from_numpy(np.zeros(self.rows, np.int32))
        self.stop = hip.DeviceArray.from_numpy(stop if stop.size else np.zeros(1, np.int32))

    def step(self, d_logits: int, row_stride: int, vocab: int, configs, d_uniforms: int,
             d_tokens: int, stream=None) -> None:
        """Enqueue one step: d_tokens[r] = the drawn id (-1 for rows done
        before it).  `configs`: SampleConfig dicts, or an array built once by
        sampler.make_configs."""
        cfgs = configs if isinstance(configs, ctypes.Array) else _configs(configs, self.rows)
        self.sampler.decode_step_device(d_logits, self.rows, row_stride, vocab, self.ring.addr,
                                        self.ring_cap, self.len.addr, self.done.addr,
                                        self.stop.addr if self.n_stop else None, self.n_stop, cfgs,
                                        d_uniforms, d_tokens, stream)

    def lengths(self) -> np.ndarray:
        hip.synchronize()
        return self.len.download()

    def finished(self) -> np.ndarray:
        hip.synchronize()
        return self.done.download() != 0

    def history(self, r: int) -> np.ndarray:
        """Row r's last min(len, ring_cap) history ids, oldest first."""
        hip.synchronize()
        n_all = int(self.len.download()[r])
        ring = self.ring.download()[r]
        n = min(n_all, self.ring_cap)
        pos = np.arange(n_all - n, n_all) % self.ring_cap
        return ring[pos].copy()

    def free(self) -> None:
        for a in (self.ring, self.len, self.done, self.stop):
            a.free()
