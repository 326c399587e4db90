'use strict';
/*
 * JavaScript restatement of hachiue's sampleLogits (src/sampler.ts:12-118),
 * runnable on Node 12 (no TypeScript syntax, no `??`).
 *
 * TEST INFRASTRUCTURE ONLY: the CPU baseline the benchmark times under Node
 * on the host cores, and a second, independent restatement the C oracle is
 * cross-checked against.  Algorithm-identical to the reference (the same
 * replace-min slot scan, Set of the last 128 history ids, stable sort,
 * binary64 arithmetic with Float32Array stores); the only change is the
 * injected uniform in place of Math.random().
 */

function option(value, fallback) {
  // `value ?? fallback`: only undefined and null take the fallback
  return value === undefined || value === null ? fallback : value;
}

/* Presence / frequency extension (no reference counterpart): for each
 * distinct history id c with count n, logits[c] = (v - frequency*n) - presence,
 * after the repetition penalty. */
function applyPresenceFrequency(logits, vocab, history, presence, frequency) {
  const counts = new Map();
  for (let i = 0; i < history.length; i++) {
    const id = history[i];
    counts.set(id, (counts.get(id) || 0) + 1);
  }
  counts.forEach(function (n, id) {
    if (id >= 0 && id < vocab) logits[id] = (logits[id] - frequency * n) - presence;
  });
}

/*
 * Returns { token, n, cutoff, ids, probs } where ids / probs are the sorted
 * candidates (for parity checks).  `logits` is mutated like the reference's.
 */
function sampleDetailed(logits, vocab, history, config, uniform) {
  const cfg = config || {};
  const temperature = option(cfg.temperature, 0.6);
  const topK = option(cfg.topK, 20);
  const topP = option(cfg.topP, 0.95);
  const minP = option(cfg.minP, 0.0);
  const repetition = option(cfg.repetitionPenalty, 1.0);
  const presence = option(cfg.presencePenalty, 0.0);
  const frequency = option(cfg.frequencyPenalty, 0.0);

  // src/sampler.ts:24-33
  if (repetition !== 1.0 && history.length > 0) {
    const recent = new Set(history.slice(-128));
    recent.forEach(function (id) {
      if (id >= 0 && id < vocab) {
        const v = logits[id];
        logits[id] = v < 0 ? v * repetition : v / repetition;
      }
    });
  }
  if ((presence !== 0 || frequency !== 0) && history.length > 0) {
    applyPresenceFrequency(logits, vocab, history, presence, frequency);
  }

  // src/sampler.ts:35-46
  if (temperature <= 0) {
    let best = 0;
    let bestValue = logits[0];
    for (let i = 1; i < vocab; i++) {
      if (logits[i] > bestValue) {
        bestValue = logits[i];
        best = i;
      }
    }
    return { token: best, n: 0, cutoff: 0, ids: [], probs: [] };
  }

  // src/sampler.ts:49-69: k slots, replace the first minimum slot
  const k = Math.max(1, Math.min(topK > 0 ? topK : 64, vocab));
  const slotIds = new Int32Array(k).fill(-1);
  const slotVals = new Float32Array(k).fill(-Infinity);
  let minSlot = 0;
  let minValue = -Infinity;
  for (let i = 0; i < vocab; i++) {
    const v = logits[i];
    if (!(v > minValue)) continue;
    slotIds[minSlot] = i;
    slotVals[minSlot] = v;
    minSlot = 0;
    minValue = slotVals[0];
    for (let j = 1; j < k; j++) {
      if (slotVals[j] < minValue) {
        minValue = slotVals[j];
        minSlot = j;
      }
    }
  }

  // src/sampler.ts:71-77: filled slots, stable sort by value, descending
  const filled = [];
  for (let j = 0; j < slotIds.length; j++) if (slotIds[j] >= 0) filled.push(j);
  filled.sort(function (a, b) { return slotVals[b] - slotVals[a]; });
  const ids = filled.map(function (j) { return slotIds[j]; });
  if (filled.length === 0) return { token: 0, n: 0, cutoff: 0, ids: ids, probs: [] };
  if (filled.length === 1) return { token: ids[0], n: 1, cutoff: 1, ids: ids, probs: [1] };

  // src/sampler.ts:79-90
  const top = slotVals[filled[0]];
  const invTemp = 1.0 / temperature;
  const probs = new Float32Array(filled.length);
  let total = 0;
  for (let i = 0; i < filled.length; i++) {
    const p = Math.exp((slotVals[filled[i]] - top) * invTemp);
    probs[i] = p;
    total += p;
  }
  for (let i = 0; i < probs.length; i++) probs[i] /= total;

  // src/sampler.ts:92-107
  const floor = minP * probs[0];
  let running = 0;
  let cutoff = probs.length;
  for (let i = 0; i < probs.length; i++) {
    if (i > 0 && probs[i] < floor) {
      cutoff = i;
      break;
    }
    running += probs[i];
    if (running >= topP) {
      cutoff = i + 1;
      break;
    }
  }

  // src/sampler.ts:109-117
  let kept = 0;
  for (let i = 0; i < cutoff; i++) kept += probs[i];
  let r = uniform * kept;
  let token = ids[cutoff - 1];
  for (let i = 0; i < cutoff; i++) {
    r -= probs[i];
    if (r <= 0) {
      token = ids[i];
      break;
    }
  }
  return { token: token, n: filled.length, cutoff: cutoff, ids: ids, probs: Array.from(probs) };
}

function sampleRow(logits, vocab, history, config, uniform) {
  return sampleDetailed(logits, vocab, history, config, uniform).token;
}

module.exports = { sampleRow: sampleRow, sampleDetailed: sampleDetailed };
