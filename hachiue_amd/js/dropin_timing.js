'use strict';
/*
 * End-to-end time of the synchronous drop-in, called as hachiue's engine
 * calls sampleLogits once per decode step (src/engine.ts:1642): one host row
 * per call, so each call copies the row to the GPU, samples it and copies the
 * token (and the penalised logits) back.
 *
 *   node dropin_timing.js <workload dir> <calls> [hip|cpu]
 *
 * The directory holds meta.json, logits.f32, uniforms.f64 and, with
 * histories, hist_ids.i32 / hist_off.f64 (as bench.py writes them).  Each
 * call gets a fresh copy of a row (the copy is not timed).  Prints one JSON
 * line: the median and mean microseconds per call.  With a backend name the
 * calls go through createSampler({ backend }) (cpu: the JavaScript sampler).
 */
const fs = require('fs');
const path = require('path');
const index = require(path.join(__dirname, 'index.js'));
const hs = process.argv[4] ? index.createSampler({ backend: process.argv[4] }) : index;

function typed(file, Ctor) {
  const buf = fs.readFileSync(file);
  const ab = new ArrayBuffer(buf.length);
  new Uint8Array(ab).set(buf);
  return new Ctor(ab);
}

const dir = process.argv[2];
const calls = parseInt(process.argv[3] || '200', 10);
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
const logits = typed(path.join(dir, 'logits.f32'), Float32Array);
const uniforms = typed(path.join(dir, 'uniforms.f64'), Float64Array);
const ids = meta.has_history ? typed(path.join(dir, 'hist_ids.i32'), Int32Array) : null;
const off = meta.has_history ? typed(path.join(dir, 'hist_off.f64'), Float64Array) : null;
function value(x) { return x === 'Infinity' ? Infinity : x === '-Infinity' ? -Infinity : x === 'NaN' ? NaN : x; }
const configs = meta.configs.map(function (c) {
  const o = {};
  Object.keys(c).forEach(function (k) { o[k] = value(c[k]); });
  return o;
});
const s = meta.stride;
const times = [];
for (let i = 0; i < calls + 10; i++) {
  const r = i % meta.rows;
  const row = logits.slice(r * s, r * s + s);
  const history = ids ? Array.from(ids.subarray(off[r], off[r + 1])) : [];
  const cfg = Object.assign({ uniform: uniforms[r] }, configs[r]);
  const t0 = process.hrtime();
  hs.sampleLogits(row, meta.vocab, history, cfg);
  const dt = process.hrtime(t0);
  if (i >= 10) times.push(dt[0] * 1e6 + dt[1] / 1e3);   // the first calls warm up
}
times.sort(function (a, b) { return a - b; });
const mean = times.reduce(function (a, b) { return a + b; }, 0) / times.length;
console.log(JSON.stringify({ calls: calls, us_median: times[times.length >> 1], us_mean: mean,
  node: process.version, backend: hs.info ? hs.info.backend : 'hip' }));
