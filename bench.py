#!/usr/bin/env python3
"""Benchmark of the gfx950 logits-to-token sampler.

One step = one full sampling pass (penalties -> top-k select -> sort ->
softmax -> min-p / top-p -> draw) over a batch of device-resident logit rows.
Default workload: 256 rows x 151936 fp32 logits, top-k 40, top-p 0.9,
repetition penalty 1.1 over a 64-token history, temperature 0.7.

Prints one JSON line: rows/s (value), ms per step, the roofline of the
dominant kernel (algorithmic bytes per launch over its average duration,
timed with HIP events on the launch stream) and a CPU
baseline (the JavaScript restatement of sampler.ts under Node on this host).

  python bench.py [--steps K] [--warmup W] [--workload NAME] [--sets N]

Other paths (one JSON line each, same fields):
  --path greedy-route   the engine's greedy route: the WGSL-order argmax over
                        the workload's logits (hs_argmax_device)
  --path lmhead         the lm_head GEMV (hs_gemv_device_ex) over a synthetic
                        vocab x hidden weight (--wfmt f32|q4_0|q4_1|q4_k|q6_k in GGUF
                        blocks, q1_0|pq2_0|ptq1_0 planar; --hidden; --hadamard)
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sampled rows/sec and HBM GB/s (% roofline) at B=256, V=151936 fp32"
HBM_PEAK_GBPS = 8000.0   # MI355X HBM3E
MALL_BYTES = 256 << 20   # MI355X last-level (Infinity) cache


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def write_workload_dir(wl, rows: int, path: str) -> None:
    """Files read by oracle/cpu_bench.js (first `rows` rows)."""
    os.makedirs(path, exist_ok=True)
    wl.logits[:rows].tofile(os.path.join(path, "logits.f32"))
    np.asarray(wl.uniforms[:rows], np.float64).tofile(os.path.join(path, "uniforms.f64"))
    has_h = wl.hist_ids is not None
    if has_h:
        end = int(wl.hist_off[rows])
        wl.hist_ids[:end].tofile(os.path.join(path, "hist_ids.i32"))
        wl.hist_off[:rows + 1].astype(np.float64).tofile(os.path.join(path, "hist_off.f64"))

    def js(v):
        if isinstance(v, float) and not np.isfinite(v):
            return "NaN" if np.isnan(v) else ("Infinity" if v > 0 else "-Infinity")
        return v

    meta = dict(rows=rows, vocab=wl.vocab, stride=wl.logits.shape[1], has_history=has_h,
                configs=[{k: js(v) for k, v in c.items()} for c in wl.configs[:rows]])
    with open(os.path.join(path, "meta.json"), "w") as f:
        json.dump(meta, f)


def cpu_baseline(wl, seconds: float, threads: int, rows: int) -> dict | None:
    """Times oracle/sampler_port.js (sampler.ts restated) under Node: one row
    of fresh logits per call, for `seconds` on 1 thread and on `threads`."""
    node = "node"
    try:
        ver = subprocess.run([node, "--version"], capture_output=True, text=True, timeout=30)
    except (OSError, subprocess.TimeoutExpired):
        return None
    if ver.returncode != 0:
        return None
    with tempfile.TemporaryDirectory(prefix="hs_cpu_") as d:
        write_workload_dir(wl, rows, d)
        cmd = [node, os.path.join(ROOT, "oracle", "cpu_bench.js"), "bench", d, str(seconds),
               str(threads)]
        log(f"[bench] cpu baseline: {' '.join(cmd[1:3])} ... {seconds}s x (1, {threads}) threads")
        out = subprocess.run(cmd, capture_output=True, text=True, timeout=seconds * 4 + 120)
    if out.returncode != 0:
        log(f"[bench] cpu baseline failed: {out.stderr[-2000:]}")
        return None
    r = json.loads(out.stdout.strip().splitlines()[-1])
    return dict(
        value=round(r["rows_per_s_all"], 1), unit="rows/s", cores=r["threads"], kind="port",
        value_1core=round(r["rows_per_s_1core"], 1), nproc=os.cpu_count(),
        sample=(f"oracle/sampler_port.js (sampler.ts restated, Node {r['node']}, {r['cpu']}): "
                f"first {rows} rows of the workload, one fresh row per call, "
                f"{seconds}s on 1 thread ({r['rows_1core']} rows) and {seconds}s on "
                f"{r['threads']} worker threads ({r['rows_all']} rows; nproc reports "
                f"{os.cpu_count()}, the GPU's host share is 16 cores); time inside the "
                f"sampler only"))


def host_api(wl, rows: int, calls: int) -> dict | None:
    """End-to-end time of the synchronous drop-in as the engine calls it
    (src/engine.ts:1642): Node sampleLogits on one host row per call (H2D of
    the row, the kernels, D2H of the token and penalised logits).  Beside it,
    the same calls on the drop-in's CPU backend (createSampler({backend:
    'cpu'}), the JavaScript sampler a host without the GPU would use)."""
    node = "node"
    addon = os.path.join(ROOT, "hachiue_amd", "node", "hachiue_sampler.node")
    if not os.path.exists(addon):
        return None
    res = {}
    with tempfile.TemporaryDirectory(prefix="hs_api_") as d:
        write_workload_dir(wl, rows, d)
        for backend in ("hip", "cpu"):
            cmd = [node, os.path.join(ROOT, "hachiue_amd", "js", "dropin_timing.js"), d,
                   str(calls), backend]
            log(f"[bench] host api ({backend}): {calls} calls")
            try:
                out = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
            except (OSError, subprocess.TimeoutExpired):
                return None
            if out.returncode != 0:
                log(f"[bench] host api timing failed: {out.stderr[-2000:]}")
                return None
            res[backend] = json.loads(out.stdout.strip().splitlines()[-1])
    r, c = res["hip"], res["cpu"]
    return dict(value=round(r["us_median"], 2), unit="us per row (median)",
                mean_us=round(r["us_mean"], 2), calls=r["calls"],
                path=(f"Node {r['node']} sampleLogits -> N-API -> hs_sample_logits: one host row "
                      f"per call (PCIe both ways), rows 0..{rows - 1} of the workload"),
                cpu_backend=dict(value=round(c["us_median"], 2), unit="us per row (median)",
                                 path="the same calls through createSampler({backend: 'cpu'}) "
                                      "(hachiue_amd/js/cpu.js, one thread)"))


def oracle_parity(wl, tokens: np.ndarray) -> dict:
    from oracle import pyoracle
    ref = wl.logits.copy()
    res = pyoracle.sample_batch(ref, wl.vocab, wl.hist_ids, wl.hist_off, wl.configs,
                                wl.uniforms)
    eq = tokens == res.token
    boundary = int(((~eq) & ((res.draw_margin < 1e-6) | (res.topp_margin < 1e-6))).sum())
    return dict(rows=int(eq.size), tokens_equal=int(eq.sum()), boundary_cases=boundary)


def load_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter on a
    device-to-device copy of known size), or None when there is none."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return int(t["traffic_bytes_per_launch"]), os.path.relpath(path, ROOT)
    except (OSError, ValueError, KeyError):
        return None, None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="headline")
    ap.add_argument("--sets", type=int, default=0,
                    help="input copies rotated per step so reads come from HBM, not MALL "
                         "(0: enough copies for twice the 256 MB last-level cache)")
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0 = min(16, cpu count): the GPU's host share")
    ap.add_argument("--api-calls", type=int, default=200,
                    help="sampleLogits calls timed end to end through Node (0: skip)")
    ap.add_argument("--cpu-rows", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--path", default="sample",
                    choices=["sample", "greedy-route", "lmhead", "lmhead-sample", "decode"])
    ap.add_argument("--wfmt", default="q6_k", help="lm_head weight format (--path lmhead)")
    ap.add_argument("--hidden", type=int, default=2048, help="lm_head K (--path lmhead)")
    ap.add_argument("--lm-fuse", default="1", choices=["0", "1", "2"],
                    help="HS_LMHEAD_FUSE of the timed context (--path lmhead-sample): 0 two "
                         "launches, 1 the library default, 2 one launch wherever it applies; "
                         "the other two are timed beside it")
    ap.add_argument("--lm-greedy", action="store_true",
                    help="--path lmhead-sample: greedy rows (temperature 0, repetition 1.1)")
    ap.add_argument("--hadamard", action="store_true",
                    help="Hadamard-folded lm_head: the input is rotated first (--path lmhead)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="end with one device-to-device copy of one input set (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (rows are "
              "independent; a batch shards by rows with no communication). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    from hachiue_amd import Sampler, hip, workloads
    from hachiue_amd.sampler import make_configs

    if args.path != "sample":
        return other_path(args)

    t_gen = time.time()
    wl = workloads.make(args.workload, seed=0)
    rows, vocab = wl.rows, wl.vocab
    log(f"[bench] workload {wl.name}: {rows} x {vocab} (generated in {time.time() - t_gen:.1f}s)")

    sampler = Sampler(0)
    stream = hip.Stream()
    cfgs = make_configs(wl.configs, rows)
    sets = args.sets if args.sets > 0 else max(1, -(-2 * MALL_BYTES // wl.logits.nbytes))
    d_logits = [hip.DeviceArray.from_numpy(wl.logits) for _ in range(sets)]
    d_ids = hip.DeviceArray.from_numpy(wl.hist_ids) if wl.hist_ids is not None else None
    d_off = hip.DeviceArray.from_numpy(wl.hist_off) if wl.hist_off is not None else None
    d_u = hip.DeviceArray.from_numpy(wl.uniforms)
    d_tok = hip.DeviceArray(rows, np.int32)

    turn = [0]   # every step reads the next input set, warm-up included

    def step(i: int) -> None:
        turn[0] += 1
        sampler.sample_device(d_logits[turn[0] % sets].addr, rows, vocab, vocab,
                              d_ids.addr if d_ids else None, d_off.addr if d_off else None,
                              cfgs, d_u.addr, d_tok.addr, stream=stream)

    parity = None
    if not args.no_parity:
        turn[0] = -1
        step(0)   # set 0
        stream.synchronize()
        parity = oracle_parity(wl, d_tok.download())
        log(f"[bench] parity vs oracle: {parity}")
        d_logits[0].upload(wl.logits)

    for i in range(args.warmup):
        step(i)
    stream.synchronize()
    log(f"[bench] warmup {args.warmup} steps done")

    def timed_region(instrumented: bool) -> tuple[float, float]:
        """K steps between a device sync and events on the launch stream."""
        sampler.set_timing(instrumented)
        sampler.kernel_times()
        e0, e1 = hip.Event(), hip.Event()
        hip.synchronize()
        e0.record(stream)
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(i)
        e1.record(stream)
        e1.synchronize()
        wall = time.perf_counter() - t0
        hip.synchronize()
        return e0.elapsed_ms(e1), wall

    # Region 1 gives `value`; region 2 repeats it with HIP events recorded
    # around each kernel launch, for the per-kernel durations of the roofline;
    # region 3 times single steps (max(K, 50)), each read back at once, for
    # the median kernel duration.
    total_ms, wall = timed_region(False)
    log(f"[bench] timed {args.steps} steps: {total_ms:.3f} ms device, {wall * 1e3:.1f} ms wall")
    inst_ms, _ = timed_region(True)
    kms, calls = sampler.kernel_times()
    log(f"[bench] instrumented {args.steps} steps: {inst_ms:.3f} ms device, kernels {kms}")
    kavg = {k: v / max(calls, 1) for k, v in kms.items()}
    dominant = max(kavg, key=kavg.get)
    sampler.set_timing(True)
    per_step, step_dev = [], []
    for i in range(max(args.steps, 50)):
        step(i)
        km, c = sampler.kernel_times()
        per_step.append(km[dominant] / max(c, 1))
        step_dev.append(sum(km.values()))   # every kernel of the step
    sampler.set_timing(False)
    kmed = float(np.median(per_step))
    log(f"[bench] {dominant}: median {kmed * 1e3:.2f} us over {len(per_step)} single steps, "
        f"mean {kavg[dominant] * 1e3:.2f} us back to back")

    ms_per_step = total_ms / args.steps
    value = rows / (ms_per_step * 1e-3)
    alg_step = wl.algorithmic_bytes()
    # The dominant kernel is credited with the step's algorithmic bytes (the
    # logits and history it streams); the other kernels move only the ids.
    achieved = alg_step / (kmed * 1e-3) / 1e9

    if args.copy_probe:   # (into a buffer of its own when there is one input set)
        dst = d_logits[1] if sets > 1 else hip.DeviceArray(wl.logits.shape, np.float32)
        dst.copy_from(d_logits[0])
        hip.synchronize()
        log(f"[bench] copy probe: {d_logits[0].nbytes} bytes device to device")

    traffic, traffic_note = load_traffic(wl.name, dominant)

    cpu = api = None
    if not args.no_cpu:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        cpu = cpu_baseline(wl, args.cpu_seconds, threads, min(args.cpu_rows, rows))
        if args.api_calls > 0:
            api = host_api(wl, min(16, rows), args.api_calls)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        # the step's device time (all its kernels, HIP events), median of
        # max(K, 50) single steps
        "ms_per_step_median": round(float(np.median(step_dev)), 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"{wl.name}: {rows} rows x {vocab} fp32 logits; "
                         + ("top-k 40, top-p 0.9, repetition 1.1 over a 64-token history, "
                            "temperature 0.7" if wl.name == "headline" else "see workloads.py")),
            "rows": rows, "vocab": vocab, "input_sets": sets,
            "algorithmic_bytes_per_step": alg_step,
        },
        "hbm_gbps_step": round(alg_step / (ms_per_step * 1e-3) / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "kernel_ms": round(kmed, 5),
            "kernel_ms_basis": f"median of {len(per_step)} single steps (HIP events)",
            "kernel_ms_mean_back_to_back": round(kavg[dominant], 5),
            "kernels_ms": {k: round(v, 5) for k, v in kavg.items() if v > 0.0005},
            "ms_per_step_instrumented": round(inst_ms / args.steps, 5),
        },
        "cpu_baseline": cpu,
        "host_api": api,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    sampler.close()
    return 0


def other_path(args) -> int:
    """The greedy-route argmax, the lm_head GEMV or the device-resident decode
    step, timed like the sampler."""
    from hachiue_amd import Sampler, hip, workloads

    def policy_context(fuse: str):
        """A context created with HS_LMHEAD_FUSE=fuse (the lm_head + sampling
        launch policy: 0 two launches, 1 the library's default, 2 one launch
        wherever it applies)."""
        os.environ["HS_LMHEAD_FUSE"] = fuse
        try:
            return Sampler(0)
        finally:
            del os.environ["HS_LMHEAD_FUSE"]

    sampler = policy_context(args.lm_fuse) if args.path == "lmhead-sample" else Sampler(0)
    stream = hip.Stream()

    def n_sets(set_bytes: int) -> int:   # as in main(): past twice the last-level cache
        return args.sets if args.sets > 0 else max(1, -(-2 * MALL_BYTES // set_bytes))
    if args.path == "greedy-route":
        wl = workloads.make(args.workload, seed=0)
        rows, vocab = wl.rows, wl.vocab
        sets = n_sets(wl.logits.nbytes)
        d_in = [hip.DeviceArray.from_numpy(wl.logits) for _ in range(sets)]
        d_tok = hip.DeviceArray(rows, np.int32)
        kernel, unit = "argmax_kernel", "rows/s"
        alg = rows * (4 * vocab + 4)
        desc = f"greedy route (WGSL-order argmax) over {wl.name}: {rows} rows x {vocab} fp32 logits"

        def step(i: int) -> None:
            sampler.argmax_device(d_in[i % sets].addr, rows, vocab, vocab, d_tok.addr, stream=stream)

        def check() -> dict:
            from oracle import pyoracle
            want = pyoracle.wgsl_argmax(wl.logits, vocab)
            got = d_tok.download()
            return {"rows": rows, "ids_equal": int((got == want).sum())}
        count = rows
    elif args.path == "decode":
        from hachiue_amd.decode import DecodeState
        wl = workloads.make(args.workload, seed=0)
        rows, vocab = wl.rows, wl.vocab
        sets = n_sets(wl.logits.nbytes)
        d_in = [hip.DeviceArray.from_numpy(wl.logits) for _ in range(sets)]
        d_u = hip.DeviceArray.from_numpy(wl.uniforms)
        d_tok = hip.DeviceArray(rows, np.int32)
        prompts = [wl.history(r) for r in range(rows)]
        state = DecodeState(sampler, prompts, stop_ids=(), ring_cap=4096)
        from hachiue_amd.sampler import make_configs
        cfgs = make_configs(wl.configs, rows)
        kernel, unit = "row_kernel", "rows/s"
        alg = wl.algorithmic_bytes()
        desc = (f"decode step (draw, stop check, history append) over {wl.name}: {rows} rows x "
                f"{vocab} fp32 logits, histories in 4096-id device rings")

        def step(i: int) -> None:
            state.step(d_in[i % sets].addr, vocab, vocab, cfgs, d_u.addr, d_tok.addr, stream=stream)

        def check() -> dict:
            from oracle import pyoracle
            ref = pyoracle.decode_loop([wl.logits.copy()], vocab, prompts, [], wl.configs,
                                       [wl.uniforms])
            got = d_tok.download()
            lens = state.lengths()
            return {"rows": rows, "tokens_equal": int((got == ref.tokens[0]).sum()),
                    "appended": int((lens == np.array([len(h) for h in ref.histories])).sum())}
        count = rows
    else:
        from hachiue_amd.sampler import PLANAR_QUANT_BYTES, split_blocks, weights
        lh = workloads.make_lmhead(args.wfmt, args.hidden)
        rows, vocab, K = lh.x.shape[0], lh.vocab, lh.hidden
        sets = n_sets(lh.weights.nbytes)
        planar = lh.wtype in PLANAR_QUANT_BYTES
        if planar:   # the reference's upload: quants and binary16 scales apart
            q, sc = split_blocks(lh.wtype, lh.weights)
            d_in = [hip.DeviceArray.from_numpy(q) for _ in range(sets)]
            d_sc = [hip.DeviceArray.from_numpy(sc) for _ in range(sets)]
        else:
            d_in = [hip.DeviceArray.from_numpy(lh.weights.reshape(-1)) for _ in range(sets)]
            d_sc = [None] * sets
        wts = [weights(lh.wtype, vocab, K, d_in[i].addr, d_sc[i].addr if d_sc[i] else None,
                       args.hadamard) for i in range(sets)]
        d_x = hip.DeviceArray.from_numpy(lh.x)
        d_y = hip.DeviceArray((rows, vocab), np.float32)
        kernel, unit = "gemv_kernel", "logit rows/s"
        alg = lh.algorithmic_bytes()
        desc = (f"lm_head GEMV: {vocab} x {K} {lh.fmt} weights ({lh.weights.nbytes} bytes, "
                f"{'planar quants + binary16 scales' if planar else 'GGUF blocks'}"
                f"{', Hadamard-folded' if args.hadamard else ''}), {rows} hidden state(s)")

        def step(i: int) -> None:
            sampler.gemv_device_ex(d_x.addr, rows, K, wts[i % sets], d_y.addr, vocab,
                                   stream=stream)

        def check() -> dict:
            from oracle import pyoracle
            got = d_y.download().astype(np.float64)
            xr = pyoracle.hadamard512(lh.x) if args.hadamard else lh.x
            exact, mag = pyoracle.gemv_exact(lh.wtype, xr, lh.weights, vocab)
            rel = np.abs(got - exact) / np.maximum(mag, 1e-30)
            return {"logits": int(got.size), "within_2^-16_of_sum_abs": int((rel <= 2 ** -16).sum()),
                    "max_rel": float(rel.max())}
        count = rows
        if args.path == "lmhead-sample":
            # the lm_head and the sampler on its rows (one launch or two, by
            # the context's policy): the headline's sampling, a 64-id
            # history per hidden state
            from hachiue_amd.sampler import make_configs
            rng = np.random.default_rng(5)
            hist = rng.integers(0, vocab, (rows, 64)).astype(np.int32)
            off = np.arange(rows + 1, dtype=np.int64) * 64
            cfg = [dict(temperature=0.0 if args.lm_greedy else 0.7, topK=40, topP=0.9,
                        repetitionPenalty=1.1)] * rows
            cfgs = make_configs(cfg, rows)
            u = rng.random(rows)
            d_ids, d_off = hip.DeviceArray.from_numpy(hist.reshape(-1)), hip.DeviceArray.from_numpy(off)
            d_u, d_t = hip.DeviceArray.from_numpy(u), hip.DeviceArray(rows, np.int32)
            unit = "sampled rows/s"
            desc = desc.replace("lm_head GEMV:", "lm_head GEMV + greedy (repetition 1.1 over 64 ids):"
                                if args.lm_greedy else
                                "lm_head GEMV + sampling (top-k 40, top-p 0.9, "
                                "repetition 1.1 over 64 ids, temperature 0.7):")

            def step_on(ctx, i: int) -> None:
                ctx.lm_head_sample_device_ex(d_x.addr, rows, K, wts[i % sets], d_y.addr, vocab,
                                             d_ids.addr, d_off.addr, cfgs, d_u.addr, d_t.addr,
                                             stream=stream)

            def step(i: int) -> None:
                step_on(sampler, i)

            def check() -> dict:
                from oracle import pyoracle
                pen = d_y.download()
                tok = d_t.download()
                sampler.gemv_device_ex(d_x.addr, rows, K, wts[0], d_y.addr, vocab, stream=stream)
                stream.synchronize()
                raw = d_y.download()
                res = pyoracle.sample_batch(raw, vocab, hist.reshape(-1), off, cfg, u)
                return {"rows": rows, "tokens_equal": int((tok == res.token).sum()),
                        "penalised_logits_equal": bool(np.array_equal(pen.view(np.uint32),
                                                                      raw.view(np.uint32)))}

    step(0)
    stream.synchronize()
    parity = None if args.no_parity else check()
    log(f"[bench] {args.path}: parity {parity}")
    for i in range(args.warmup):
        step(i)
    stream.synchronize()

    def region(instrumented: bool) -> float:
        sampler.set_timing(instrumented)
        sampler.kernel_times()
        e0, e1 = hip.Event(), hip.Event()
        hip.synchronize()
        e0.record(stream)
        for i in range(args.steps):
            step(i)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1)

    total_ms = region(False)
    region(True)
    kms, _ = sampler.kernel_times()
    sampler.set_timing(False)
    # per step: a step is one call, of one launch or two (the GEMV, then the
    # sampler), each counted as a timed call
    kms_avg = kms[kernel] / args.steps
    by_policy = None
    if args.path == "lmhead-sample":
        # the same calls on a context of each policy, timed in three rounds
        # with the policies in rotated order (whichever runs last in a round
        # measured about 2 us faster), the median of the rounds
        ctxs = {args.lm_fuse: sampler}
        for fuse in ("0", "1", "2"):
            if fuse not in ctxs:
                ctxs[fuse] = policy_context(fuse)
                for i in range(args.warmup):
                    step_on(ctxs[fuse], i)
        hip.synchronize()
        order = sorted(ctxs)
        per = {f: [] for f in order}
        for rnd in range(3):
            for fuse in order[rnd:] + order[:rnd]:
                e0, e1 = hip.Event(), hip.Event()
                e0.record(stream)
                for i in range(args.steps):
                    step_on(ctxs[fuse], i)
                e1.record(stream)
                e1.synchronize()
                per[fuse].append(e0.elapsed_ms(e1) / args.steps)
        by_policy = {f: round(float(np.median(per[f])), 5) for f in order}
        for fuse, ctx in ctxs.items():
            if fuse != args.lm_fuse:
                ctx.close()
        log("[bench] lmhead-sample: us per step by HS_LMHEAD_FUSE (rotated rounds) " +
            ", ".join(f"{k}: {by_policy[k] * 1e3:.2f}" for k in sorted(by_policy)))
    if args.copy_probe and sets > 1:   # a copy of known size for the counters' scale
        d_in[1].copy_from(d_in[0])
        hip.synchronize()
        log(f"[bench] copy probe: {d_in[0].nbytes} bytes device to device")
    ms_per_step = total_ms / args.steps
    achieved = alg / (kms_avg * 1e-3) / 1e9
    # measured HBM traffic of the matrix-core K-quant GEMV at its committed shape
    traffic, traffic_note = None, None
    if (args.path == "lmhead" and rows == 1 and not args.hadamard and lh.fmt in ("q4_k", "q6_k")):
        traffic, traffic_note = load_traffic(f"lmhead_{lh.fmt.replace('_', '')}_{vocab}x{K}",
                                             "gemv_kq_mfma_kernel")
    line = {
        "metric": f"{args.path}: {unit} and HBM GB/s (% roofline)",
        "value": round(count / (ms_per_step * 1e-3), 1),
        "unit": unit,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": desc, "rows": rows, "vocab": vocab, "input_sets": sets,
                   "algorithmic_bytes_per_step": alg},
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_note, "kernel_ms": round(kms_avg, 5)},
        "cpu_baseline": None,
        "parity": parity,
    }
    if by_policy is not None:
        line["config"]["lm_head_fuse"] = args.lm_fuse
        line["ms_per_step_by_fuse_policy"] = {k: by_policy[k] for k in sorted(by_policy)}
        line["kernels_ms"] = {k: round(v / args.steps, 5) for k, v in kms.items() if v > 0}
    print(json.dumps(line), flush=True)
    sampler.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
