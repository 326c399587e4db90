'use strict';
/*
 * CPU baseline / cross-check driver for sampler_port.js (TEST INFRASTRUCTURE
 * ONLY).  Reads a workload directory written by the benchmark or the tests:
 *   meta.json      {rows, vocab, stride, configs: [...], has_history}
 *   logits.f32     rows*stride float32
 *   hist_ids.i32   concatenated int32 history ids      (if has_history)
 *   hist_off.f64   rows+1 offsets as float64            (if has_history)
 *   uniforms.f64   rows float64
 *
 *   node cpu_bench.js check <dir> [cap]       one JSON line per row
 *   node cpu_bench.js kat <cases.json>        the known-answer cases, one line each
 *   node cpu_bench.js bench <dir> <seconds> <threads> [max_rows]
 *
 * bench: like the engine (src/engine.ts:1642) each call gets one row of
 * fresh logits (a copy, not timed); the time inside sampleRow is summed.
 */
const fs = require('fs');
const os = require('os');
const path = require('path');
const wt = require('worker_threads');
const port = require('./sampler_port.js');

function typed(file, Ctor) {
  const buf = fs.readFileSync(file);
  const ab = new ArrayBuffer(buf.length);
  new Uint8Array(ab).set(buf);
  return new Ctor(ab);
}

function load(dir) {
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const w = { meta: meta };
  w.logits = typed(path.join(dir, 'logits.f32'), Float32Array);
  w.uniforms = typed(path.join(dir, 'uniforms.f64'), Float64Array);
  if (meta.has_history) {
    w.histIds = typed(path.join(dir, 'hist_ids.i32'), Int32Array);
    w.histOff = typed(path.join(dir, 'hist_off.f64'), Float64Array);
  }
  w.configs = meta.configs.map(function (c) {
    const out = {};
    Object.keys(c).forEach(function (key) {
      const v = c[key];
      out[key] = v === 'Infinity' ? Infinity : v === '-Infinity' ? -Infinity : v === 'NaN' ? NaN : v;
    });
    return out;
  });
  return w;
}

function history(w, r) {
  if (!w.histIds) return [];
  return Array.from(w.histIds.subarray(w.histOff[r], w.histOff[r + 1]));
}

function rowCopy(w, r) {
  const s = w.meta.stride;
  return w.logits.slice(r * s, r * s + s);
}

function check(dir, cap) {
  const w = load(dir);
  const lines = [];
  for (let r = 0; r < w.meta.rows; r++) {
    const row = rowCopy(w, r);
    const out = port.sampleDetailed(row, w.meta.vocab, history(w, r), w.configs[r], w.uniforms[r]);
    lines.push(JSON.stringify({
      token: out.token, n: out.n, cutoff: out.cutoff,
      ids: out.ids.slice(0, cap), probs: out.probs.slice(0, cap),
      logits_sum: Array.from(row.subarray(0, w.meta.vocab)).reduce(function (a, b) { return a + (isFinite(b) ? b : 0); }, 0),
    }));
  }
  process.stdout.write(lines.join('\n') + '\n');
}

function special(x) {
  if (x === 'NaN') return NaN;
  if (x === 'Infinity') return Infinity;
  if (x === '-Infinity') return -Infinity;
  if (x === '-0') return -0;
  return x;
}

function kat(file) {
  const data = JSON.parse(fs.readFileSync(file, 'utf8'));
  const out = [];
  data.cases.forEach(function (c) {
    const logits = new Float32Array(c.logits.map(special));
    const cfg = {};
    Object.keys(c.config).forEach(function (key) { cfg[key] = special(c.config[key]); });
    const r = port.sampleDetailed(logits, c.vocab, c.history.slice(), cfg, c.u);
    out.push(JSON.stringify({
      name: c.name, token: r.token, n: r.n, cutoff: r.cutoff, ids: r.ids, probs: r.probs,
      logits_bits: Array.from(new Uint32Array(logits.buffer)),
    }));
  });
  process.stdout.write(out.join('\n') + '\n');
}

function runFor(w, seconds, first, step, maxRows) {
  const rows = Math.min(w.meta.rows, maxRows || w.meta.rows);
  const hist = [];
  for (let r = 0; r < rows; r++) hist.push(history(w, r));
  let done = 0;
  let busyNs = 0n;
  const deadline = process.hrtime.bigint() + BigInt(Math.round(seconds * 1e9));
  let r = first;
  let sink = 0;
  while (process.hrtime.bigint() < deadline) {
    const row = rowCopy(w, r);
    const t0 = process.hrtime.bigint();
    sink += port.sampleRow(row, w.meta.vocab, hist[r], w.configs[r], w.uniforms[r]);
    busyNs += process.hrtime.bigint() - t0;
    done++;
    r += step;
    if (r >= rows) r = first % step;
  }
  return { rows: done, busy_s: Number(busyNs) / 1e9, sink: sink };
}

function bench(dir, seconds, threads, maxRows) {
  const single = runFor(load(dir), seconds, 0, 1, maxRows);
  const one = single.rows / single.busy_s;
  if (threads <= 1) {
    report(one, single.rows, one, single.rows, 1, seconds);
    return;
  }
  let pending = threads;
  let total = 0;
  let totalRows = 0;
  for (let t = 0; t < threads; t++) {
    const worker = new wt.Worker(__filename, {
      workerData: { dir: dir, seconds: seconds, first: t, step: threads, maxRows: maxRows },
    });
    worker.on('message', function (m) {
      total += m.rows / m.busy_s;
      totalRows += m.rows;
    });
    worker.on('error', function (e) { throw e; });
    worker.on('exit', function () {
      if (--pending === 0) report(one, single.rows, total, totalRows, threads, seconds);
    });
  }
}

function report(one, oneRows, all, allRows, threads, seconds) {
  const cpus = os.cpus();
  process.stdout.write(JSON.stringify({
    rows_per_s_1core: one, rows_1core: oneRows,
    rows_per_s_all: all, rows_all: allRows, threads: threads, seconds: seconds,
    node: process.version, cpu: cpus.length ? cpus[0].model : 'unknown',
  }) + '\n');
}

if (!wt.isMainThread) {
  const d = wt.workerData;
  const res = runFor(load(d.dir), d.seconds, d.first, d.step, d.maxRows);
  wt.parentPort.postMessage(res);
} else if (require.main === module) {
  const mode = process.argv[2];
  if (mode === 'check') check(process.argv[3], Number(process.argv[4] || 64));
  else if (mode === 'kat') kat(process.argv[3]);
  else if (mode === 'bench')
    bench(process.argv[3], Number(process.argv[4] || 5), Number(process.argv[5] || 1),
      Number(process.argv[6] || 0));
  else {
    process.stderr.write('usage: cpu_bench.js check <dir> [cap] | kat <cases.json> | bench <dir> <seconds> <threads> [max_rows]\n');
    process.exit(2);
  }
}
