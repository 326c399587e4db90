'use strict';
// Drives hachiue_amd/js (the sampleLogits drop-in) for the tests:
//   node dropin_check.js kat <cases.json>
//   node dropin_check.js rows <workload dir>     sampleLogits row by row
//   node dropin_check.js batch <workload dir>    sampleLogitsBatch (+ async)
//   node dropin_check.js argmax <workload dir>   argmaxLogits / argmaxLogitsBatch / nextToken
//   node dropin_check.js route                   isGreedyRoute on option objects
//   node dropin_check.js nogpu                   error behaviour without a GPU
//   node dropin_check.js concurrent <dir>        two async batches in flight together with
//                                                sync calls on the shared default context
//   node dropin_check.js rule <cases.json>       drawRule's decision per case (no GPU)
//   node dropin_check.js draws <cases.json>      Math.random() calls and tokens of
//                                                sampleLogits / sampleLogitsBatch
//   node dropin_check.js greedy <cases.json>     argmaxLogits / nextToken on hand cases
//   node dropin_check.js backend <name>          createSampler's choice and its info
//   node dropin_check.js cpu-candidates <dir>    cpu.js sampleLogitsCandidates row by row
const fs = require('fs');
const path = require('path');
const mod = require(path.join(__dirname, '..', '..', 'hachiue_amd', 'js', 'index.js'));
// HS_BACKEND=cpu|auto|hip runs the modes through createSampler on that backend
const hs = process.env.HS_BACKEND ? mod.createSampler({ backend: process.env.HS_BACKEND }) : mod;

function special(x) {
  return x === 'NaN' ? NaN : x === 'Infinity' ? Infinity : x === '-Infinity' ? -Infinity
    : x === '-0' ? -0 : x;
}
function typed(file, Ctor) {
  const buf = fs.readFileSync(file);
  const ab = new ArrayBuffer(buf.length);
  new Uint8Array(ab).set(buf);
  return new Ctor(ab);
}
function load(dir) {
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const w = { meta: meta, logits: typed(path.join(dir, 'logits.f32'), Float32Array),
    uniforms: typed(path.join(dir, 'uniforms.f64'), Float64Array) };
  if (meta.has_history) {
    w.ids = typed(path.join(dir, 'hist_ids.i32'), Int32Array);
    w.off = typed(path.join(dir, 'hist_off.f64'), Float64Array);
  }
  w.configs = meta.configs.map(function (c) {
    const o = {};
    Object.keys(c).forEach(function (k) { o[k] = special(c[k]); });
    return o;
  });
  w.history = function (r) { return w.ids ? Array.from(w.ids.subarray(w.off[r], w.off[r + 1])) : []; };
  return w;
}
function bits(a) { return Array.from(new Uint32Array(a.buffer, a.byteOffset, a.length)); }

const mode = process.argv[2];
if (mode === 'kat') {
  const data = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
  data.cases.forEach(function (c) {
    const logits = new Float32Array(c.logits.map(special));
    const cfg = { uniform: c.u };
    Object.keys(c.config).forEach(function (k) { cfg[k] = special(c.config[k]); });
    const token = hs.sampleLogits(logits, c.vocab, c.history.slice(), cfg);
    console.log(JSON.stringify({ name: c.name, token: token, logits_bits: bits(logits) }));
  });
} else if (mode === 'rows') {
  const w = load(process.argv[3]);
  const s = w.meta.stride;
  for (let r = 0; r < w.meta.rows; r++) {
    const row = w.logits.slice(r * s, r * s + s);
    const cfg = Object.assign({ uniform: w.uniforms[r] }, w.configs[r]);
    const token = hs.sampleLogits(row, w.meta.vocab, w.history(r), cfg);
    console.log(JSON.stringify({ row: r, token: token }));
  }
} else if (mode === 'batch') {
  const w = load(process.argv[3]);
  const hists = w.ids ? w.configs.map(function (_, r) { return w.history(r); }) : null;
  const logits = w.logits.slice();
  const tok = hs.sampleLogitsBatch(logits, w.meta.vocab, hists, w.configs, w.uniforms,
    { rows: w.meta.rows, stride: w.meta.stride });
  const logits2 = w.logits.slice();
  hs.sampleLogitsBatchAsync(logits2, w.meta.vocab, hists, w.configs, w.uniforms,
    { rows: w.meta.rows, stride: w.meta.stride }).then(function (tok2) {
    console.log(JSON.stringify({ tokens: Array.from(tok), tokens_async: Array.from(tok2),
      logits_same: bits(logits).join() === bits(logits2).join(),
      penalised: bits(logits) }));
  }, function (e) { console.error(e); process.exit(1); });
} else if (mode === 'concurrent') {
  const w = load(process.argv[3]);
  const hists = w.ids ? w.configs.map(function (_, r) { return w.history(r); }) : null;
  const shape = { rows: w.meta.rows, stride: w.meta.stride };
  const a = w.logits.slice();
  const b = w.logits.slice();
  const pa = hs.sampleLogitsBatchAsync(a, w.meta.vocab, hists, w.configs, w.uniforms, shape);
  const pb = hs.sampleLogitsBatchAsync(b, w.meta.vocab, hists, w.configs, w.uniforms, shape);
  // sync calls while both batches are in flight on the same context
  const s = w.meta.stride;
  const rows = [];
  for (let r = 0; r < w.meta.rows; r++) {
    const row = w.logits.slice(r * s, r * s + s);
    rows.push(hs.sampleLogits(row, w.meta.vocab, w.history(r),
      Object.assign({ uniform: w.uniforms[r] }, w.configs[r])));
  }
  Promise.all([pa, pb]).then(function (t) {
    console.log(JSON.stringify({ a: Array.from(t[0]), b: Array.from(t[1]), rows: rows,
      a_bits: bits(a), b_same: bits(a).join() === bits(b).join() }));
  }, function (e) { console.error(e); process.exit(1); });
} else if (mode === 'argmax') {
  const w = load(process.argv[3]);
  const s = w.meta.stride;
  const before = bits(w.logits).join();
  const batch = hs.argmaxLogitsBatch(w.logits, w.meta.vocab, { rows: w.meta.rows, stride: s });
  const rows = [];
  const next = [];
  for (let r = 0; r < w.meta.rows; r++) {
    const row = w.logits.slice(r * s, r * s + w.meta.vocab);
    rows.push(hs.argmaxLogits(row, w.meta.vocab));
    next.push(hs.nextToken(row, w.meta.vocab, [], { temperature: 0 }));
  }
  console.log(JSON.stringify({ batch: Array.from(batch), rows: rows, next: next,
    unchanged: bits(w.logits).join() === before }));
} else if (mode === 'route') {
  const cases = [undefined, {}, { temperature: 0 }, { temperature: -1 }, { temperature: null },
    { temperature: 0, repetitionPenalty: 1.0 }, { temperature: 0, repetitionPenalty: 1.1 },
    { temperature: 0, repetitionPenalty: null }, { temperature: 0.5 }, { temperature: NaN }];
  console.log(JSON.stringify(cases.map(hs.isGreedyRoute)));
} else if (mode === 'rule' || mode === 'draws') {
  const data = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
  const FIELDS = ['temperature', 'topK', 'topP', 'minP', 'repetitionPenalty',
    'presencePenalty', 'frequencyPenalty'];
  const DEF = [0.6, 20, 0.95, 0, 1, 0, 0];
  const real = Math.random;
  let calls = 0;
  Math.random = function () { calls++; return 0.5; };
  const rows = data.cases.map(function (c) {
    const cfg = {};
    Object.keys(c.config).forEach(function (k) { cfg[k] = special(c.config[k]); });
    const logits = new Float32Array(c.logits.map(special));
    if (mode === 'rule') {
      const packed = new Float64Array(FIELDS.map(function (f, i) {
        return cfg[f] === undefined ? DEF[i] : cfg[f];
      }));
      const ids = new Int32Array(c.history);
      return { name: c.name, rule: mod.drawRule(packed, 0, c.vocab, logits, 0, c.vocab, ids, 0, ids.length) };
    }
    calls = 0;
    const token = hs.sampleLogits(logits, c.vocab, c.history.slice(), cfg);
    return { name: c.name, token: token, calls: calls };
  });
  if (mode === 'draws') {
    // the same cases as one batch (rows padded with -Infinity to one stride)
    const V = Math.max.apply(null, data.cases.map(function (c) { return c.vocab; }));
    const all = new Float32Array(V * data.cases.length).fill(-Infinity);
    data.cases.forEach(function (c, r) { all.set(new Float32Array(c.logits.map(special)), r * V); });
    const cfgs = data.cases.map(function (c) {
      const o = {};
      Object.keys(c.config).forEach(function (k) { o[k] = special(c.config[k]); });
      return o;
    });
    calls = 0;
    const tok = hs.sampleLogitsBatch(all, V, data.cases.map(function (c) { return c.history; }), cfgs,
      null, { rows: data.cases.length, stride: V });
    rows.push({ name: '(batch)', tokens: Array.from(tok), calls: calls });
  }
  Math.random = real;
  rows.forEach(function (r) { console.log(JSON.stringify(r)); });
} else if (mode === 'greedy') {
  const data = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
  data.cases.forEach(function (c) {
    const logits = new Float32Array(c.logits.map(special));
    const before = bits(logits).join();
    const id = hs.argmaxLogits(logits, c.vocab);
    const next = hs.nextToken(logits, c.vocab, [], { temperature: 0 });
    const batch = hs.argmaxLogitsBatch(logits, c.vocab, { rows: 1, stride: c.vocab })[0];
    console.log(JSON.stringify({ name: c.name, id: id, next: next, batch: batch,
      unchanged: bits(logits).join() === before }));
  });
} else if (mode === 'cpu-candidates') {
  // the CPU backend's candidate lists, row by row
  const cpu = require(path.join(__dirname, '..', '..', 'hachiue_amd', 'js', 'cpu.js'));
  const w = load(process.argv[3]);
  const s = w.meta.stride;
  for (let r = 0; r < w.meta.rows; r++) {
    const row = w.logits.slice(r * s, r * s + s);
    const cfg = Object.assign({ uniform: w.uniforms[r] }, w.configs[r]);
    const o = cpu.sampleLogitsCandidates(row, w.meta.vocab, w.history(r), cfg);
    console.log(JSON.stringify({ row: r, token: o.token, ids: Array.from(o.ids),
      probs: bits(o.probs), cutoff: o.cutoff }));
  }
} else if (mode === 'backend') {
  const out = {};
  try {
    const b = mod.createSampler({ backend: process.argv[3] });
    out.info = b.info;
    out.token = b.sampleLogits(new Float32Array([1, 3, 2]), 3, [], { temperature: 0 });
  } catch (e) {
    out.error = e.code || e.name;
  }
  console.log(JSON.stringify(out));
} else if (mode === 'nogpu') {
  const out = {};
  out.vocab0 = hs.sampleLogits(new Float32Array([1, 2]), 0, [], {});
  try {
    hs.sampleLogits(new Float32Array([1, 2, 3]), 3, [0], { temperature: 1 });
    out.error = null;
  } catch (e) {
    out.error = e.code || e.message;
  }
  try { hs.sampleLogits([1, 2, 3], 3, [], {}); } catch (e) { out.type_error = e instanceof TypeError; }
  console.log(JSON.stringify(out));
}
