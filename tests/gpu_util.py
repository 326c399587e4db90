"""Helpers shared by the GPU parity tests: run a workload through the device
C ABI and compare every output with the CPU oracle."""
from __future__ import annotations

import sys
from dataclasses import dataclass

import numpy as np

from hachiue_amd import hip
from hachiue_amd.sampler import make_configs
from oracle import pyoracle

# Parity bar: probabilities within 1e-5 relative (fp32 softmax); a token may
# differ only when the draw lands within 1e-6 of a cumulative boundary, and a
# cutoff only when the running sum is within 1e-6 of topP.
PROB_RTOL = 1e-5
BOUNDARY = 1e-6


@dataclass
class GpuResult:
    tokens: np.ndarray
    cand_ids: np.ndarray
    cand_probs: np.ndarray
    n: np.ndarray
    cutoff: np.ndarray
    flags: np.ndarray
    logits: np.ndarray


def run_gpu(sampler, logits, vocab, hist_ids, hist_off, configs, uniforms, cap=64,
            stride=None, want_cands=True) -> GpuResult:
    """want_cands=False asks for no candidate ids or probabilities (the
    kernels may then skip ordering the whole candidate list); the returned
    cand_ids / cand_probs are None."""
    rows = logits.shape[0]
    stride = logits.shape[1] if stride is None else stride
    print(f"[gpu] rows={rows} vocab={vocab} stride={stride} cap={cap} cands={want_cands}",
          flush=True)
    d_logits = hip.DeviceArray.from_numpy(logits)
    d_ids = hip.DeviceArray.from_numpy(hist_ids) if hist_ids is not None else None
    d_off = hip.DeviceArray.from_numpy(hist_off) if hist_off is not None else None
    d_u = hip.DeviceArray.from_numpy(np.asarray(uniforms, np.float64))
    d_tok = hip.DeviceArray(rows, np.int32)
    d_cid = hip.DeviceArray((rows, cap), np.int32)
    d_cpr = hip.DeviceArray((rows, cap), np.float32)
    d_n = hip.DeviceArray(rows, np.int32)
    d_cut = hip.DeviceArray(rows, np.int32)
    d_fl = hip.DeviceArray(rows, np.uint32)
    cfgs = make_configs(configs, rows)
    sampler.sample_device(d_logits.addr, rows, stride, vocab, d_ids.addr if d_ids else None,
                          d_off.addr if d_off else None, cfgs, d_u.addr, d_tok.addr,
                          cand_stride=cap, d_cand_ids=d_cid.addr if want_cands else None,
                          d_cand_probs=d_cpr.addr if want_cands else None,
                          d_cand_count=d_n.addr, d_cutoff=d_cut.addr, d_row_flags=d_fl.addr)
    hip.synchronize()
    return GpuResult(d_tok.download(), d_cid.download() if want_cands else None,
                     d_cpr.download() if want_cands else None, d_n.download(),
                     d_cut.download(), d_fl.download(), d_logits.download())


def run_oracle(logits, vocab, hist_ids, hist_off, configs, uniforms, cap=64):
    ref = logits.copy()
    res = pyoracle.sample_batch(ref, vocab, hist_ids, hist_off, configs,
                                np.asarray(uniforms, np.float64), pyoracle.HEAP, cap)
    return res, ref


def compare(got: GpuResult, want, want_logits, configs, vocab, cap, label=""):
    """Assert parity; returns the number of boundary cases tolerated."""
    rows = got.tokens.shape[0]
    if isinstance(configs, dict) or configs is None:
        configs = [configs] * rows
    same = got.logits.view(np.uint32) == want_logits.view(np.uint32)
    bad = np.flatnonzero(~same.reshape(rows, -1).all(axis=1))
    assert bad.size == 0, f"{label}: penalised logits differ in rows {bad[:10]}"
    boundary = 0
    probs_total = probs_exact = 0
    errors = []
    for r in range(rows):
        path = int(want.path[r])
        if path == 0:   # greedy
            if got.tokens[r] != want.token[r]:
                errors.append(f"row {r}: greedy {got.tokens[r]} != {want.token[r]}")
            continue
        n = int(want.n[r])
        if got.n[r] != n:
            errors.append(f"row {r}: candidate count {got.n[r]} != {n}")
            continue
        m = min(n, cap)
        if got.cand_ids is None:
            pass   # tokens, counts and cutoffs only
        elif not np.array_equal(got.cand_ids[r, :m], want.cand_ids[r, :m]):
            errors.append(f"row {r}: candidate ids differ "
                          f"{got.cand_ids[r, :8].tolist()} vs {want.cand_ids[r, :8].tolist()}")
        if n >= 2 and got.cand_probs is not None:
            gp, wp = got.cand_probs[r, :m].astype(np.float64), want.cand_probs[r, :m].astype(np.float64)
            with np.errstate(invalid="ignore"):
                rel = np.abs(gp - wp) / np.maximum(np.abs(wp), np.finfo(np.float32).tiny)
            # a +Infinity candidate makes every probability NaN in the
            # reference too ((Inf - Inf) * invTemp, src/sampler.ts:84)
            ok = (rel <= PROB_RTOL) | (np.isnan(gp) & np.isnan(wp))
            probs_total += m
            probs_exact += int(((gp == wp) | (np.isnan(gp) & np.isnan(wp))).sum())
            if not ok.all():
                errors.append(f"row {r}: probs rel err {np.nanmax(rel):.3g}")
        near_topp = want.topp_margin[r] < BOUNDARY
        if got.cutoff[r] != want.cutoff[r] and not near_topp:
            errors.append(f"row {r}: cutoff {got.cutoff[r]} != {want.cutoff[r]}")
        if got.tokens[r] != want.token[r]:
            if want.draw_margin[r] < BOUNDARY or near_topp:
                boundary += 1
            else:
                errors.append(f"row {r}: token {got.tokens[r]} != {want.token[r]} "
                              f"(draw margin {want.draw_margin[r]:.3g})")
    assert not errors, f"{label}: {len(errors)} mismatches: " + "; ".join(errors[:8])
    print(f"[parity] {label}: {rows} rows ok, boundary cases {boundary}, "
          f"probabilities bit-equal {probs_exact}/{probs_total}", file=sys.stderr)
    return boundary
