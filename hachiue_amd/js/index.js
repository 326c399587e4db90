'use strict';
/*
 * MI355X (gfx950) drop-in for hachiue's CPU sampler.
 *
 * sampleLogits(logits, vocab, history, config) keeps the signature, option
 * names, `??` defaults, in-place penalties and return values of
 * src/sampler.ts:12-118 (exported at src/index.ts:15); the work runs in the
 * HIP kernels behind the C ABI (include/hachiue_sampler.h) through the
 * Node-API addon.  There is no CPU fallback: without the addon or a GPU the
 * first call throws.
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

// Math.random() is reached only with a positive temperature and more than
// one slot (src/sampler.ts:36, :49, :77).
function mayDraw(cfg, offset, vocab) {
  if (!(cfg[offset] > 0)) return false;
  const t = cfg[offset + 1] > 0 ? cfg[offset + 1] : 64;
  return Math.max(1, Math.min(t, vocab)) >= 2;
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
  let u = config ? option(config.uniform, null) : null;
  if (u === null) u = mayDraw(cfg, 0, vocab) ? Math.random() : 0;
  const n = scanLength(vocab);
  const ids = historyIds(history);
  if (n <= logits.length) return native().sampleRow(context(), logits, n, ids, cfg, u);
  // indices past the array read `undefined` in the reference, which no
  // comparison selects: pad with NaN and copy the penalised values back
  const padded = new Float32Array(n).fill(NaN);
  padded.set(logits);
  const token = native().sampleRow(context(), padded, n, ids, cfg, u);
  logits.set(padded.subarray(0, logits.length));
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
  const u = new Float64Array(rows);
  for (let r = 0; r < rows; r++) {
    const given = uniforms ? uniforms[r] : undefined;
    u[r] = given !== undefined && given !== null ? given
      : (mayDraw(cfg, FIELDS.length * r, vocab) ? Math.random() : 0);
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
  return [context(), logits, rows, stride, vocab, ids, off, cfg, u];
}

/**
 * Many rows in one call: logits holds `rows` rows of `stride` floats
 * (default stride = vocab); histories[r], configs[r] (or one shared config)
 * and uniforms[r] (or Math.random() when the reference would draw).
 * @returns {Int32Array} tokens
 */
function sampleLogitsBatch(logits, vocab, histories, configs, uniforms, shape) {
  const a = batchArgs(logits, vocab, histories, configs, uniforms, shape);
  return native().sampleBatch.apply(null, a);
}

/** Promise-returning variant of sampleLogitsBatch (runs off the main thread). */
function sampleLogitsBatchAsync(logits, vocab, histories, configs, uniforms, shape) {
  const a = batchArgs(logits, vocab, histories, configs, uniforms, shape);
  return native().sampleBatchAsync.apply(null, a);
}

module.exports = {
  sampleLogits: sampleLogits,
  sampleLogitsBatch: sampleLogitsBatch,
  sampleLogitsBatchAsync: sampleLogitsBatchAsync,
  isGreedyRoute: isGreedyRoute,
  argmaxLogits: argmaxLogits,
  argmaxLogitsBatch: argmaxLogitsBatch,
  nextToken: nextToken,
  DEFAULTS: Object.freeze({
    temperature: 0.6, topK: 20, topP: 0.95, minP: 0.0, repetitionPenalty: 1.0,
  }),
};
