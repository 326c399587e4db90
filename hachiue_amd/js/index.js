'use strict';
/*
 * MI355X (gfx950) drop-in for hachiue's CPU sampler.
 *
 * sampleLogits(logits, vocab, history, config) keeps the signature, option
 * names, `??` defaults, in-place penalties and return values of
 * src/sampler.ts:12-118 (exported at src/index.ts:15); the work runs in the
 * HIP kernels behind the C ABI (include/hachiue_sampler.h) through the
 * Node-API addon.  These module-level functions never fall back to the CPU:
 * without the addon or a GPU the first call throws (code 'HS_ERR_HIP').
 *
 * createSampler({ backend }) picks a backend the way the engine does
 * (src/engine.ts:521, :556-557, :626-639): 'hip' (the default here) throws
 * when the HIP backend cannot start; 'cpu' takes the JavaScript sampler of
 * cpu.js; 'auto' takes HIP when it starts and the CPU otherwise, with the
 * reason in info.fallbackReason.
 *
 * Extensions (absent by default, so existing callers see no change):
 *   config.presencePenalty / config.frequencyPenalty  (x - freq*n) - pres
 *   config.uniform   the value in [0, 1) used instead of Math.random()
 *   sampleLogitsBatch / sampleLogitsBatchAsync        many rows per call
 *
 * The engine's greedy route (src/engine.ts:1600-1601): with temperature <= 0
 * and no repetition penalty the engine takes the token from the WGSL argmax
 * of its forward pass (src/kernels.ts:1613-1654), not from sampleLogits.
 *   isGreedyRoute(options)               that decision
 *   argmaxLogits / argmaxLogitsBatch     that argmax, with its tie order
 *   nextToken(logits, vocab, history, options)   the engine's choice between
 *                                        the two (src/engine.ts:1616-1620, :1642-1646)
 */
const path = require('path');

const FIELDS = ['temperature', 'topK', 'topP', 'minP', 'repetitionPenalty',
  'presencePenalty', 'frequencyPenalty'];
// src/sampler.ts:18-22; the extensions default to 0
const DEFAULTS = [0.6, 20, 0.95, 0.0, 1.0, 0.0, 0.0];

let addon = null;
function native() {
  if (addon === null) addon = require(path.join(__dirname, '..', 'node', 'hachiue_sampler.node'));
  return addon;
}

let defaultContext = null;
function context() {
  if (defaultContext === null) defaultContext = native().createContext(0);
  return defaultContext;
}

function option(value, fallback) {
  // `value ?? fallback`
  return value === undefined || value === null ? fallback : value;
}

// SampleConfig -> 7 numbers (hs_sample_config order) at out[offset..]
function packConfig(config, vocab, out, offset) {
  const c = config || {};
  for (let i = 0; i < FIELDS.length; i++) out[offset + i] = Number(option(c[FIELDS[i]], DEFAULTS[i]));
  if (!Number.isInteger(vocab)) {
    // k = max(1, min(topK > 0 ? topK : 64, vocab)) with a fractional vocab:
    // clamp here, the library scans ceil(vocab) logits like the reference
    const t = out[offset + 1] > 0 ? out[offset + 1] : 64;
    out[offset + 1] = Math.min(t, vocab);
  }
}

// Whether sampleLogits would call Math.random() for a row (src/sampler.ts:
// 36, :49-50, :76-77, :112): once iff !(temperature <= 0) (a NaN temperature
// draws) and order.length >= 2, where order.length = min(k, the number of
// penalised logits > -Infinity).  Penalties touch only history ids, so two
// logits > -Infinity at ids outside the history settle it before the call.
// Returns 1 (draws), 0 (does not) or -1 (only the penalised row can tell).
const DRAW = 1;
const NO_DRAW = 0;
const DRAW_UNKNOWN = -1;
function drawRule(cfg, offset, vocab, logits, base, n, ids, h0, h1) {
  if (cfg[offset] <= 0) return NO_DRAW;
  const t = cfg[offset + 1] > 0 ? cfg[offset + 1] : 64;
  if (Math.trunc(Math.max(1, Math.min(t, vocab))) < 2) return NO_DRAW;
  const rep = cfg[offset + 4] !== 1;
  const pf = cfg[offset + 5] !== 0 || cfg[offset + 6] !== 0;
  // ids a penalty may change: the last 128 entries for the repetition
  // penalty alone, the whole history with presence / frequency
  const lo = pf ? h0 : Math.max(h0, h1 - 128);
  const touched = (rep || pf) && h1 > lo;
  let set = null;
  let checks = 0;
  let found = 0;
  for (let i = 0; i < n; i++) {
    if (!(logits[base + i] > -Infinity)) continue;
    if (touched) {
      let hit;
      if (set !== null) hit = set.has(i);
      else if (++checks <= 8) hit = ids.subarray(lo, h1).indexOf(i) >= 0;
      else {
        set = new Set(ids.subarray(lo, h1));
        hit = set.has(i);
      }
      if (hit) continue;
    }
    if (++found === 2) return DRAW;
  }
  return touched ? DRAW_UNKNOWN : NO_DRAW;
}

// order.length >= 2 on a penalised row (k >= 2 known)
function twoCandidates(logits, base, n) {
  let found = 0;
  for (let i = 0; i < n; i++) if (logits[base + i] > -Infinity && ++found === 2) return true;
  return false;
}

// The same configs with the penalties switched off, for a second pass over
// logits that already hold the penalised values.
function withoutPenalties(cfg) {
  const out = Float64Array.from(cfg);
  for (let o = 0; o < out.length; o += FIELDS.length) {
    out[o + 4] = 1;
    out[o + 5] = 0;
    out[o + 6] = 0;
  }
  return out;
}

// Ids that index nothing in the reference (non-integers, out of int32) -> -1.
function historyIds(history) {
  if (history instanceof Int32Array) return history;
  const h = history || [];
  const out = new Int32Array(h.length);
  for (let i = 0; i < h.length; i++) {
    const x = h[i];
    out[i] = Number.isInteger(x) && x >= -2147483648 && x <= 2147483647 ? x : -1;
  }
  return out;
}

function scanLength(vocab) {
  return Number.isInteger(vocab) ? vocab : Math.ceil(vocab);
}

/**
 * Drop-in for sampleLogits (src/sampler.ts:12-17).
 * @param {Float32Array} logits  updated in place with the penalised values
 * @param {number} vocab
 * @param {number[]|Int32Array} history
 * @param {object} [config]
 * @returns {number} token id
 */
function sampleLogits(logits, vocab, history, config) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  if (!(vocab > 0)) return 0;   // no logit is read; every path returns 0
  const cfg = new Float64Array(FIELDS.length);
  packConfig(config, vocab, cfg, 0);
  const n = scanLength(vocab);
  const ids = historyIds(history);
  // indices past the array read `undefined` in the reference, which no
  // comparison selects: pad with NaN and copy the penalised values back
  const row = n <= logits.length ? logits : new Float32Array(n).fill(NaN);
  if (row !== logits) row.set(logits);
  const given = config ? option(config.uniform, null) : null;
  let token;
  const rule = given !== null ? DRAW : drawRule(cfg, 0, vocab, row, 0, n, ids, 0, ids.length);
  if (rule !== DRAW_UNKNOWN) {
    const u = given !== null ? given : (rule === DRAW ? Math.random() : 0);
    token = native().sampleRow(context(), row, n, ids, cfg, u);
  } else {
    // a penalty decides whether two candidates remain: penalise and sample
    // without a draw, then draw on the penalised row only if it has them
    token = native().sampleRow(context(), row, n, ids, cfg, 0);
    if (twoCandidates(row, 0, n)) {
      token = native().sampleRow(context(), row, n, new Int32Array(0), withoutPenalties(cfg),
        Math.random());
    }
  }
  if (row !== logits) logits.set(row.subarray(0, logits.length));
  return token;
}

/**
 * src/engine.ts:1600-1601: greedy decoding without a repetition penalty takes
 * the GPU argmax instead of sampleLogits.
 * @param {object} [options]
 * @returns {boolean}
 */
function isGreedyRoute(options) {
  const o = options || {};
  return option(o.temperature, 0.6) <= 0 &&
    (o.repetitionPenalty === undefined || o.repetitionPenalty === 1.0);
}

/**
 * The WGSL argmax of src/kernels.ts:1613-1654 over `rows` rows of `stride`
 * floats (default: one row, stride = vocab).  Its tie order differs from
 * sampleLogits' greedy path: among equal maxima the id whose low byte,
 * bit-reversed, is smallest wins, then the smallest id; NaN and values at or
 * below -1e30 are never taken (0 when nothing else is).  Logits are read only.
 * @returns {Int32Array} ids
 */
function argmaxLogitsBatch(logits, vocab, shape) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  if (!Number.isInteger(vocab) || vocab < 0) throw new RangeError('vocab must be a non-negative integer');
  const stride = (shape && shape.stride) || vocab;
  const rows = (shape && shape.rows !== undefined) ? shape.rows
    : (stride > 0 ? Math.floor(logits.length / stride) : 0);
  return native().argmax(context(), logits, rows, stride, vocab);
}

/** One row of argmaxLogitsBatch: the engine's greedy token. */
function argmaxLogits(logits, vocab) {
  return argmaxLogitsBatch(logits, vocab, { rows: 1, stride: vocab })[0];
}

/**
 * The engine's next token (src/engine.ts:1616-1620, :1642-1646): the GPU
 * argmax on its greedy route, sampleLogits otherwise.
 */
function nextToken(logits, vocab, history, options) {
  return isGreedyRoute(options) ? argmaxLogits(logits, vocab)
    : sampleLogits(logits, vocab, history, options);
}

function batchArgs(logits, vocab, histories, configs, uniforms, shape) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  if (!Number.isInteger(vocab) || vocab < 0) throw new RangeError('vocab must be a non-negative integer');
  const stride = (shape && shape.stride) || vocab;
  const rows = (shape && shape.rows !== undefined) ? shape.rows
    : (stride > 0 ? Math.floor(logits.length / stride) : 0);
  const cfg = new Float64Array(FIELDS.length * rows);
  for (let r = 0; r < rows; r++) {
    const c = Array.isArray(configs) ? configs[r] : configs;
    packConfig(c, vocab, cfg, FIELDS.length * r);
  }
  let ids = null;
  let off = null;
  if (histories) {
    off = new Float64Array(rows + 1);
    const parts = [];
    for (let r = 0; r < rows; r++) {
      const h = historyIds(histories[r]);
      parts.push(h);
      off[r + 1] = off[r] + h.length;
    }
    ids = new Int32Array(off[rows] || 1);
    for (let r = 0; r < rows; r++) ids.set(parts[r], off[r]);
  }
  // one Math.random() per row that draws, in row order; a row whose draw
  // only its penalised values decide leaves the rest to a second pass
  const u = new Float64Array(rows);
  const rules = new Int8Array(rows);
  let unknown = false;
  for (let r = 0; r < rows; r++) {
    const given = uniforms ? uniforms[r] : undefined;
    if (given !== undefined && given !== null) {
      u[r] = given;
      rules[r] = DRAW;
      continue;
    }
    rules[r] = vocab > 0 ? drawRule(cfg, FIELDS.length * r, vocab, logits, r * stride, vocab,
      ids, off ? off[r] : 0, off ? off[r + 1] : 0) : NO_DRAW;
    if (rules[r] === DRAW_UNKNOWN) unknown = true;
  }
  if (!unknown) {
    for (let r = 0; r < rows; r++) if (rules[r] === DRAW && !(uniforms && uniforms[r] != null)) u[r] = Math.random();
  }
  const args = [context(), logits, rows, stride, vocab, ids, off, cfg, u];
  if (!unknown) return { args: args, second: null };
  // pass 1 penalises with no draw; the draws then follow the penalised rows
  const second = function () {
    const u2 = new Float64Array(rows);
    for (let r = 0; r < rows; r++) {
      const given = uniforms ? uniforms[r] : undefined;
      if (given !== undefined && given !== null) u2[r] = given;
      else if (rules[r] === DRAW || (rules[r] === DRAW_UNKNOWN && twoCandidates(logits, r * stride, vocab))) {
        u2[r] = Math.random();
      }
    }
    return [context(), logits, rows, stride, vocab, null, null, withoutPenalties(cfg), u2];
  };
  return { args: args, second: second };
}

/**
 * Many rows in one call: logits holds `rows` rows of `stride` floats
 * (default stride = vocab); histories[r], configs[r] (or one shared config)
 * and uniforms[r] (or Math.random(), called once for each row that draws,
 * in row order, under sampleLogits' rule).
 * @returns {Int32Array} tokens
 */
function sampleLogitsBatch(logits, vocab, histories, configs, uniforms, shape) {
  const a = batchArgs(logits, vocab, histories, configs, uniforms, shape);
  const tokens = native().sampleBatch.apply(null, a.args);
  return a.second === null ? tokens : native().sampleBatch.apply(null, a.second());
}

/** Promise-returning variant of sampleLogitsBatch (runs off the main thread). */
function sampleLogitsBatchAsync(logits, vocab, histories, configs, uniforms, shape) {
  const a = batchArgs(logits, vocab, histories, configs, uniforms, shape);
  const p = native().sampleBatchAsync.apply(null, a.args);
  return a.second === null ? p
    : p.then(function () { return native().sampleBatchAsync.apply(null, a.second()); });
}

const API = ['sampleLogits', 'sampleLogitsBatch', 'sampleLogitsBatchAsync', 'isGreedyRoute',
  'argmaxLogits', 'argmaxLogitsBatch', 'nextToken'];

function backendObject(impl, info) {
  const b = { info: Object.freeze(info) };
  API.forEach(function (name) { b[name] = impl[name]; });
  return Object.freeze(b);
}

/**
 * A sampler on the requested backend: 'hip' (default), 'cpu' or 'auto'.
 * The result has the module's functions and `info` = { backend, label,
 * fallbackReason? } (BackendInfo, src/engine.ts:532-539).
 */
function createSampler(options) {
  const requested = option(options && options.backend, 'hip');
  if (requested === 'cpu') return backendObject(require('./cpu.js'), { backend: 'cpu', label: 'CPU (JavaScript)' });
  if (requested !== 'hip' && requested !== 'auto') {
    throw new TypeError("backend must be 'hip', 'cpu' or 'auto'");
  }
  try {
    context();
  } catch (err) {
    if (requested === 'hip') throw err;
    const reason = err instanceof Error ? err.message : String(err);
    return backendObject(require('./cpu.js'),
      { backend: 'cpu', label: 'CPU (JavaScript)', fallbackReason: reason });
  }
  return backendObject(module.exports, { backend: 'hip', label: 'HIP (gfx950)' });
}

module.exports = {
  createSampler: createSampler,
  sampleLogits: sampleLogits,
  sampleLogitsBatch: sampleLogitsBatch,
  sampleLogitsBatchAsync: sampleLogitsBatchAsync,
  isGreedyRoute: isGreedyRoute,
  argmaxLogits: argmaxLogits,
  argmaxLogitsBatch: argmaxLogitsBatch,
  nextToken: nextToken,
  drawRule: drawRule,
  DEFAULTS: Object.freeze({
    temperature: 0.6, topK: 20, topP: 0.95, minP: 0.0, repetitionPenalty: 1.0,
  }),
};
