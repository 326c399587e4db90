'use strict';
/*
 * CPU backend of the sampler, for hosts where the HIP library or a GPU is
 * absent: sampleLogits (src/sampler.ts:12-118, with this library's
 * presence/frequency extension) and the greedy loop of the reference's Wasm
 * backend (src/wasm-backend.ts:1204-1215), in plain JavaScript.
 *
 * It is reached only by asking for it: createSampler({ backend: 'cpu' }), or
 * backend 'auto' after the HIP backend failed to start (the engine's fallback
 * from WebGPU to Wasm, src/engine.ts:626-639).  The module-level functions of
 * index.js never fall back.
 *
 * Selection.  The reference keeps k slots and, for every logit above the
 * current minimum, overwrites the first slot holding that minimum and
 * rescans (src/sampler.ts:50-69), an O(V * k) loop on rows with many
 * entries.  Here the slots sit in a binary heap ordered by (value, slot):
 * its root is exactly the slot the rescan finds (the smallest value, the
 * lowest slot among equal ones), so the same logit lands in the same slot
 * in O(log k).  Until k slots are filled the minimum is -Infinity and every
 * logit above it takes the next empty slot, so the fill is a plain copy.
 * The stable descending sort (src/sampler.ts:72-75) is value descending,
 * slot ascending; it runs as one numeric sort of packed (value, slot) keys.
 */

const FIELDS = ['temperature', 'topK', 'topP', 'minP', 'repetitionPenalty',
  'presencePenalty', 'frequencyPenalty'];
const DEFAULTS = [0.6, 20, 0.95, 0.0, 1.0, 0.0, 0.0];

function option(value, fallback) {
  // `value ?? fallback`
  return value === undefined || value === null ? fallback : value;
}

function resolve(config) {
  const c = config || {};
  const out = new Array(FIELDS.length);
  for (let i = 0; i < FIELDS.length; i++) out[i] = option(c[FIELDS[i]], DEFAULTS[i]);
  return out;
}

// src/sampler.ts:24-33: every distinct id of the last 128 history entries,
// scaled once in place.  The statement is applied as JavaScript applies it to
// a Float32Array, so ids that are not array indices change nothing.
function repetition(logits, vocab, history, p) {
  if (p !== 1.0 && history.length > 0) {
    const seen = new Set(Array.prototype.slice.call(history, -128));
    seen.forEach(function (id) {
      if (id >= 0 && id < vocab) {
        const v = logits[id];
        logits[id] = v < 0 ? v * p : v / p;
      }
    });
  }
}

// Extension: over the whole history, logit = f32((v - freq * n) - pres) for
// every int32 id in range with count n, after the repetition penalty.
function presenceFrequency(logits, vocab, history, pres, freq) {
  if (!(pres !== 0 || freq !== 0) || history.length === 0) return;
  const counts = new Map();
  for (let i = 0; i < history.length; i++) {
    const id = history[i];
    if (Number.isInteger(id) && id >= 0 && id < vocab && id <= 2147483647) {
      counts.set(id, (counts.get(id) || 0) + 1);
    }
  }
  counts.forEach(function (n, id) {
    logits[id] = (logits[id] - freq * n) - pres;
  });
}

// first index of the largest logit, strict '>' from logits[0]
// (src/sampler.ts:36-46)
function firstMax(logits, n) {
  let best = 0;
  let bv = logits[0];
  for (let i = 1; i < n; i++) {
    const v = logits[i];
    if (v > bv) {
      bv = v;
      best = i;
    }
  }
  return best;
}

// ---- the slot heap: slot indices ordered by (value, slot)
function less(val, a, b) {
  const x = val[a];
  const y = val[b];
  return x < y || (!(y < x) && a < b);
}

function siftDown(heap, val, size, at) {
  const s = heap[at];
  for (;;) {
    let c = 2 * at + 1;
    if (c >= size) break;
    if (c + 1 < size && less(val, heap[c + 1], heap[c])) c++;
    if (!less(val, heap[c], s)) break;
    heap[at] = heap[c];
    at = c;
  }
  heap[at] = s;
}

const f32 = new Float32Array(1);
const u32 = new Uint32Array(f32.buffer);
const SLOT_BITS = 2097152;   // 2^21 slots: (32-bit key, slot) stays below 2^53

// 0 for the largest value; equal values (+0 and -0 too) share a key
function descKey(v) {
  f32[0] = v === 0 ? 0 : v;
  const u = u32[0];
  const asc = u >= 0x80000000 ? (~u >>> 0) : (u + 0x80000000);
  return 0xFFFFFFFF - asc;
}

// the filled slots, value descending and slot ascending
function sortedSlots(val, filled) {
  const order = new Int32Array(filled);
  if (filled <= SLOT_BITS) {
    const keys = new Float64Array(filled);
    for (let s = 0; s < filled; s++) keys[s] = descKey(val[s]) * SLOT_BITS + s;
    keys.sort();
    for (let i = 0; i < filled; i++) order[i] = keys[i] % SLOT_BITS;
    return order;
  }
  const tmp = Array.from({ length: filled }, function (_, s) { return s; });
  tmp.sort(function (a, b) {
    const x = val[a];
    const y = val[b];
    return y > x ? 1 : y < x ? -1 : a - b;
  });
  for (let i = 0; i < filled; i++) order[i] = tmp[i];
  return order;
}

// One row already penalised: the token, calling draw() at most once, when
// the reference calls Math.random().  With `out`, also the sorted candidate
// ids and probabilities and the cutoff (out.ids, out.probs, out.cutoff).
function sampleRow(logits, vocab, temp, topK, topP, minP, draw, out) {
  const n = Math.min(Math.ceil(vocab), logits.length);
  if (temp <= 0) return n > 0 ? firstMax(logits, n) : 0;

  // src/sampler.ts:49: the slot count (typed arrays truncate a fractional k);
  // slots beyond the scanned logits can never fill
  const kr = Math.max(1, Math.min(topK > 0 ? topK : 64, vocab));
  const k = Math.min(kr >= 0 ? Math.floor(kr) : 0, n);
  if (!(k > 0)) return 0;
  const ids = new Int32Array(k);
  const val = new Float32Array(k);

  // fill: while a slot is empty the minimum is -Infinity
  let filled = 0;
  let i = 0;
  for (; i < n && filled < k; i++) {
    const v = logits[i];
    if (v > -Infinity) {
      ids[filled] = i;
      val[filled] = v;
      filled++;
    }
  }
  if (filled === k && i < n) {
    const heap = new Int32Array(k);
    for (let s = 0; s < k; s++) heap[s] = s;
    for (let at = (k >> 1) - 1; at >= 0; at--) siftDown(heap, val, k, at);
    let minVal = val[heap[0]];
    for (; i < n; i++) {
      const v = logits[i];
      if (v > minVal) {
        const s = heap[0];
        ids[s] = i;
        val[s] = v;
        siftDown(heap, val, k, 0);
        minVal = val[heap[0]];
      }
    }
  }

  if (filled === 0) return 0;
  const order = sortedSlots(val, filled);
  if (out) {
    out.ids = new Int32Array(filled);
    for (let j = 0; j < filled; j++) out.ids[j] = ids[order[j]];
  }
  if (filled === 1) return ids[order[0]];

  // src/sampler.ts:79-117: binary64 arithmetic, binary32 stores
  const m = filled;
  const maxLogit = val[order[0]];
  const invTemp = 1.0 / temp;
  const probs = new Float32Array(m);
  let sumProb = 0;
  for (let j = 0; j < m; j++) {
    const p = Math.exp((val[order[j]] - maxLogit) * invTemp);
    probs[j] = p;
    sumProb += p;
  }
  for (let j = 0; j < m; j++) probs[j] = probs[j] / sumProb;

  const minThreshold = minP * probs[0];
  let cumProb = 0;
  let cutoff = m;
  for (let j = 0; j < m; j++) {
    if (j > 0 && probs[j] < minThreshold) {
      cutoff = j;
      break;
    }
    cumProb += probs[j];
    if (cumProb >= topP) {
      cutoff = j + 1;
      break;
    }
  }
  if (out) {
    out.probs = probs;
    out.cutoff = cutoff;
  }
  let keptSum = 0;
  for (let j = 0; j < cutoff; j++) keptSum += probs[j];
  let r = draw() * keptSum;
  for (let j = 0; j < cutoff; j++) {
    r -= probs[j];
    if (r <= 0) return ids[order[j]];
  }
  return ids[order[cutoff - 1]];
}

function sampleInPlace(logits, vocab, history, c, draw, out) {
  const h = history || [];
  repetition(logits, vocab, h, c[4]);
  presenceFrequency(logits, vocab, h, Number(c[5]), Number(c[6]));
  return sampleRow(logits, vocab, c[0], c[1], c[2], c[3], draw, out);
}

function drawFrom(uniform) {
  return uniform === null ? Math.random : function () { return uniform; };
}

/**
 * sampleLogits (src/sampler.ts:12-17) on the CPU: same arguments, in-place
 * penalties and return values; config.uniform replaces Math.random().
 */
function sampleLogits(logits, vocab, history, config) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  if (!(vocab > 0)) return 0;
  const u = config ? option(config.uniform, null) : null;
  return sampleInPlace(logits, vocab, history, resolve(config), drawFrom(u));
}

/**
 * sampleLogits with its candidate list (the CPU side of
 * hs_sample_batch_device_ex's outputs): { token, ids, probs, cutoff }, ids
 * and probs in the sorted order (value descending, slot ascending), probs
 * empty when fewer than two candidates remain or on the greedy path.
 */
function sampleLogitsCandidates(logits, vocab, history, config) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  const out = { token: 0, ids: new Int32Array(0), probs: new Float32Array(0), cutoff: 0 };
  if (!(vocab > 0)) return out;
  const u = config ? option(config.uniform, null) : null;
  out.token = sampleInPlace(logits, vocab, history, resolve(config), drawFrom(u), out);
  return out;
}

// the batch shape, checked as the HIP backend checks it
function rowsOf(logits, vocab, shape) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  if (!Number.isInteger(vocab) || vocab < 0) throw new RangeError('vocab must be a non-negative integer');
  const stride = (shape && shape.stride) || vocab;
  const rows = (shape && shape.rows !== undefined) ? shape.rows
    : (stride > 0 ? Math.floor(logits.length / stride) : 0);
  if (!Number.isInteger(rows) || rows < 0) throw new RangeError('rows must be a non-negative integer');
  if (!Number.isInteger(stride) || stride < vocab) throw new RangeError('stride must be an integer >= vocab');
  if (rows > 0 && (rows - 1) * stride + vocab > logits.length) {
    throw new RangeError('logits holds fewer than rows x stride floats');
  }
  return { rows: rows, stride: stride };
}

/**
 * Many rows (sampleLogitsBatch's arguments), one after another in row order:
 * histories[r], configs[r] (or one shared config), uniforms[r] (or
 * Math.random(), called for each row that draws, in row order).
 */
function sampleLogitsBatch(logits, vocab, histories, configs, uniforms, shape) {
  const s = rowsOf(logits, vocab, shape);
  const tokens = new Int32Array(s.rows);
  if (vocab === 0) return tokens;
  const shared = Array.isArray(configs) ? null : resolve(configs);
  for (let r = 0; r < s.rows; r++) {
    const row = logits.subarray(r * s.stride, r * s.stride + vocab);
    const c = shared || resolve(configs[r]);
    const u = uniforms ? option(uniforms[r], null) : null;
    tokens[r] = sampleInPlace(row, vocab, histories ? histories[r] : null, c, drawFrom(u));
  }
  return tokens;
}

function sampleLogitsBatchAsync(logits, vocab, histories, configs, uniforms, shape) {
  try {
    return Promise.resolve(sampleLogitsBatch(logits, vocab, histories, configs, uniforms, shape));
  } catch (e) {
    return Promise.reject(e);
  }
}

/**
 * The Wasm backend's greedy route (src/wasm-backend.ts:1204-1215): the first
 * id of the largest logit above -1e30 (compared in binary64), 0 when none
 * is.  Logits are read only.
 */
function argmaxLogits(logits, vocab) {
  if (!(logits instanceof Float32Array)) throw new TypeError('logits must be a Float32Array');
  let bestVal = -1e30;
  let bestIdx = 0;
  const n = Math.min(Math.ceil(vocab), logits.length);
  for (let i = 0; i < n; i++) {
    const v = logits[i];
    if (v > bestVal) {
      bestVal = v;
      bestIdx = i;
    }
  }
  return bestIdx;
}

function argmaxLogitsBatch(logits, vocab, shape) {
  const s = rowsOf(logits, vocab, shape);
  const out = new Int32Array(s.rows);
  for (let r = 0; r < s.rows; r++) {
    out[r] = argmaxLogits(logits.subarray(r * s.stride, r * s.stride + vocab), vocab);
  }
  return out;
}

/** src/engine.ts:1600-1601: temperature <= 0 and no repetition penalty. */
function isGreedyRoute(options) {
  const o = options || {};
  return option(o.temperature, 0.6) <= 0 &&
    (o.repetitionPenalty === undefined || o.repetitionPenalty === 1.0);
}

/** The engine's choice on this backend: the greedy loop, or sampleLogits. */
function nextToken(logits, vocab, history, options) {
  return isGreedyRoute(options) ? argmaxLogits(logits, vocab)
    : sampleLogits(logits, vocab, history, options);
}

module.exports = {
  sampleLogits: sampleLogits,
  sampleLogitsCandidates: sampleLogitsCandidates,
  sampleLogitsBatch: sampleLogitsBatch,
  sampleLogitsBatchAsync: sampleLogitsBatchAsync,
  isGreedyRoute: isGreedyRoute,
  argmaxLogits: argmaxLogits,
  argmaxLogitsBatch: argmaxLogitsBatch,
  nextToken: nextToken,
};
