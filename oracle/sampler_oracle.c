/*
 * CPU restatement of hachiue's sampleLogits (src/sampler.ts:12-118).
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker for the HIP sampler.  Only the
 * tests, the smoke check and the benchmark's CPU-baseline leg load it.
 *
 * Number model (the reference runs in JavaScript): a Float32Array element
 * read is an exact binary64 value; all arithmetic is binary64; a store into a
 * Float32Array rounds to nearest-even binary32.  Built with
 * -ffp-contract=off so no fused multiply-add changes a rounding.
 */
#include "sampler_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* src/sampler.ts:49  k = Math.max(1, Math.min(topK > 0 ? topK : 64, vocab)),
 * then `new Int32Array(k)` (ToIndex) truncates a fractional length. */
int64_t orc_resolve_k(double top_k, int64_t vocab) {
  double t = (top_k > 0) ? top_k : 64.0; /* NaN > 0 is false -> 64 */
  double m = t < (double)vocab ? t : (double)vocab;
  double k = m > 1.0 ? m : 1.0;
  return (int64_t)floor(k);
}

static int cmp_i32(const void *a, const void *b) {
  int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
  return (x > y) - (x < y);
}

/* src/sampler.ts:24-33: `new Set(history.slice(-128))`, each distinct id in
 * [0, vocab) scaled once: v < 0 ? v * p : v / p (binary64), stored binary32.
 * Extension (no reference counterpart): for each distinct id c of the whole
 * history with count n, logits[c] = f32((v - freq * n) - pres).  Applied
 * after the repetition penalty. */
void orc_apply_penalties(float *logits, int64_t vocab, const int32_t *hist,
                         int64_t hist_len, const orc_config *cfg) {
  const double rp = cfg->repetition_penalty;
  if (rp != 1.0 && hist_len > 0) {
    int64_t start = hist_len > 128 ? hist_len - 128 : 0;
    int64_t n = hist_len - start;
    int32_t tmp[128];
    memcpy(tmp, hist + start, (size_t)n * sizeof(int32_t));
    qsort(tmp, (size_t)n, sizeof(int32_t), cmp_i32); /* set semantics: order irrelevant */
    for (int64_t i = 0; i < n; ++i) {
      if (i > 0 && tmp[i] == tmp[i - 1]) continue;
      int32_t id = tmp[i];
      if (id >= 0 && id < vocab) {
        double v = (double)logits[id];
        logits[id] = (float)(v < 0 ? v * rp : v / rp);
      }
    }
  }
  const double pres = cfg->presence_penalty, freq = cfg->frequency_penalty;
  if ((pres != 0.0 || freq != 0.0) && hist_len > 0) {
    int32_t *tmp = (int32_t *)malloc((size_t)hist_len * sizeof(int32_t));
    if (!tmp) return;
    memcpy(tmp, hist, (size_t)hist_len * sizeof(int32_t));
    qsort(tmp, (size_t)hist_len, sizeof(int32_t), cmp_i32);
    for (int64_t i = 0; i < hist_len;) {
      int64_t j = i;
      while (j < hist_len && tmp[j] == tmp[i]) ++j;
      int32_t id = tmp[i];
      if (id >= 0 && id < vocab) {
        double x = (double)logits[id];
        x = x - freq * (double)(j - i);
        x = x - pres;
        logits[id] = (float)x;
      }
      i = j;
    }
    free(tmp);
  }
}

/* src/sampler.ts:35-46: first index of the maximum, strict '>' from logits[0]. */
static int32_t greedy_argmax(const float *logits, int64_t vocab) {
  int32_t best = 0;
  float bv = logits[0];
  for (int64_t i = 1; i < vocab; ++i) {
    if (logits[i] > bv) {
      bv = logits[i];
      best = (int32_t)i;
    }
  }
  return best;
}

/* src/sampler.ts:50-69, verbatim: k slots; a value enters iff it is strictly
 * greater than the current minimum, into the FIRST slot holding that minimum
 * (strict '<' rescan from slot 0). */
static void topk_literal(const float *logits, int64_t vocab, int64_t k,
                         int32_t *ids, float *vals) {
  for (int64_t j = 0; j < k; ++j) {
    ids[j] = -1;
    vals[j] = -INFINITY;
  }
  int64_t mi = 0;
  float mv = -INFINITY;
  for (int64_t i = 0; i < vocab; ++i) {
    float v = logits[i];
    if (v > mv) {
      ids[mi] = (int32_t)i;
      vals[mi] = v;
      mi = 0;
      mv = vals[0];
      for (int64_t j = 1; j < k; ++j) {
        if (vals[j] < mv) {
          mv = vals[j];
          mi = j;
        }
      }
    }
  }
}

/* Same semantics with the first-minimum slot kept at the top of a binary
 * heap ordered by (value, slot index): the heap top is exactly the slot the
 * rescan above would find, so the final slots are identical.  O(V + R log k). */
static int heap_less(const float *vals, int32_t a, int32_t b) {
  return vals[a] < vals[b] || (vals[a] == vals[b] && a < b);
}

static void topk_heap(const float *logits, int64_t vocab, int64_t k,
                      int32_t *ids, float *vals, int32_t *heap) {
  for (int64_t j = 0; j < k; ++j) {
    ids[j] = -1;
    vals[j] = -INFINITY;
    heap[j] = (int32_t)j; /* all -Inf: ordered by slot index, a valid heap */
  }
  for (int64_t i = 0; i < vocab; ++i) {
    float v = logits[i];
    int32_t top = heap[0];
    if (!(v > vals[top])) continue;
    ids[top] = (int32_t)i;
    vals[top] = v;
    int64_t pos = 0;
    for (;;) {
      int64_t l = 2 * pos + 1, r = l + 1, m = pos;
      if (l < k && heap_less(vals, heap[l], heap[m])) m = l;
      if (r < k && heap_less(vals, heap[r], heap[m])) m = r;
      if (m == pos) break;
      int32_t t = heap[pos];
      heap[pos] = heap[m];
      heap[m] = t;
      pos = m;
    }
  }
}

int orc_topk_slots(const float *logits, int64_t vocab, int64_t k, int method,
                   int32_t *slot_ids, float *slot_vals) {
  if (method == ORC_TOPK_LITERAL) {
    topk_literal(logits, vocab, k, slot_ids, slot_vals);
    return 0;
  }
  int32_t *heap = (int32_t *)malloc((size_t)k * sizeof(int32_t));
  if (!heap) return -1;
  topk_heap(logits, vocab, k, slot_ids, slot_vals, heap);
  free(heap);
  return 0;
}

/* Stable merge sort of slot indices by value, descending.  The reference sorts
 * with (a, b) => vals[b] - vals[a]; Array.prototype.sort is stable (ES2019),
 * so equal values keep ascending slot order. */
static void stable_sort_desc(int32_t *idx, int32_t *tmp, int64_t n,
                             const float *vals) {
  for (int64_t w = 1; w < n; w *= 2) {
    for (int64_t lo = 0; lo < n; lo += 2 * w) {
      int64_t mid = lo + w < n ? lo + w : n;
      int64_t hi = lo + 2 * w < n ? lo + 2 * w : n;
      int64_t a = lo, b = mid, o = lo;
      while (a < mid && b < hi) {
        /* take from the right run only if strictly greater */
        if (vals[idx[b]] > vals[idx[a]]) tmp[o++] = idx[b++];
        else tmp[o++] = idx[a++];
      }
      while (a < mid) tmp[o++] = idx[a++];
      while (b < hi) tmp[o++] = idx[b++];
    }
    memcpy(idx, tmp, (size_t)n * sizeof(int32_t));
  }
}

int orc_sample_row(float *logits, int64_t vocab, const int32_t *hist,
                   int64_t hist_len, const orc_config *cfg, double u,
                   int method, orc_result *res, int32_t *cand_ids,
                   float *cand_vals, float *cand_probs, int64_t cap) {
  memset(res, 0, sizeof(*res));
  res->draw_margin = INFINITY;
  res->topp_margin = INFINITY;
  res->draw_index = -1;

  orc_apply_penalties(logits, vocab, hist, hist_len, cfg);

  const double temp = cfg->temperature;
  if (temp <= 0) { /* src/sampler.ts:36 */
    res->path = 0;
    res->token = vocab > 0 ? greedy_argmax(logits, vocab) : 0;
    return 0;
  }

  const int64_t k = orc_resolve_k(cfg->top_k, vocab);
  res->k = (int32_t)k;
  int32_t *ids = (int32_t *)malloc((size_t)k * sizeof(int32_t));
  float *vals = (float *)malloc((size_t)k * sizeof(float));
  int32_t *order = (int32_t *)malloc((size_t)k * sizeof(int32_t));
  int32_t *tmp = (int32_t *)malloc((size_t)k * sizeof(int32_t));
  float *probs = (float *)malloc((size_t)k * sizeof(float));
  if (!ids || !vals || !order || !tmp || !probs) {
    free(ids); free(vals); free(order); free(tmp); free(probs);
    return -1;
  }
  if (method == ORC_TOPK_LITERAL) topk_literal(logits, vocab, k, ids, vals);
  else topk_heap(logits, vocab, k, ids, vals, tmp);

  /* src/sampler.ts:72-74: slots with an id, stable-sorted by value desc */
  int64_t n = 0;
  for (int64_t j = 0; j < k; ++j)
    if (ids[j] >= 0) order[n++] = (int32_t)j;
  stable_sort_desc(order, tmp, n, vals);
  res->n = (int32_t)n;
  for (int64_t i = 0; i < n && i < cap; ++i) {
    if (cand_ids) cand_ids[i] = ids[order[i]];
    if (cand_vals) cand_vals[i] = vals[order[i]];
  }

  if (n == 0) { /* src/sampler.ts:76 */
    res->path = 1;
    res->token = 0;
  } else if (n == 1) { /* src/sampler.ts:77: no draw */
    res->path = 2;
    res->token = ids[order[0]];
    res->cutoff = 1;
    res->draw_index = 0;
    if (cand_probs && cap > 0) cand_probs[0] = 1.0f;
  } else {
    /* src/sampler.ts:79-90 */
    const double max_logit = (double)vals[order[0]];
    const double inv_temp = 1.0 / temp;
    double sum = 0;
    for (int64_t i = 0; i < n; ++i) {
      double p = exp(((double)vals[order[i]] - max_logit) * inv_temp);
      probs[i] = (float)p;
      sum += p;
    }
    for (int64_t i = 0; i < n; ++i) probs[i] = (float)((double)probs[i] / sum);
    res->sum_prob = sum;

    /* src/sampler.ts:93-107 */
    const double min_thr = cfg->min_p * (double)probs[0];
    double cum = 0;
    int64_t cutoff = n;
    for (int64_t i = 0; i < n; ++i) {
      if (i > 0 && (double)probs[i] < min_thr) {
        cutoff = i;
        break;
      }
      cum += (double)probs[i];
      double dm = fabs(cum - cfg->top_p);
      if (dm < res->topp_margin) res->topp_margin = dm;
      if (cum >= cfg->top_p) {
        cutoff = i + 1;
        break;
      }
    }

    /* src/sampler.ts:109-117 */
    double kept = 0;
    for (int64_t i = 0; i < cutoff; ++i) kept += (double)probs[i];
    double r = u * kept;
    const double r0 = r;
    int64_t pick = cutoff - 1;
    double c2 = 0;
    int found = 0;
    for (int64_t i = 0; i < cutoff; ++i) {
      c2 += (double)probs[i];
      double dm = fabs(r0 - c2);
      if (dm < res->draw_margin) res->draw_margin = dm;
      if (!found) {
        r -= (double)probs[i];
        if (r <= 0) {
          pick = i;
          found = 1;
        }
      }
    }
    res->path = 3;
    res->cutoff = (int32_t)cutoff;
    res->kept_sum = kept;
    res->draw_index = (int32_t)pick;
    res->token = ids[order[pick]];
    if (cand_probs)
      for (int64_t i = 0; i < n && i < cap; ++i) cand_probs[i] = probs[i];
  }
  free(ids); free(vals); free(order); free(tmp); free(probs);
  return 0;
}

int orc_sample_batch(float *logits, int64_t rows, int64_t stride, int64_t vocab,
                     const int32_t *hist_ids, const int64_t *hist_off,
                     const orc_config *cfgs, const double *u, int method,
                     orc_result *res, int32_t *cand_ids, float *cand_vals,
                     float *cand_probs, int64_t cap) {
  for (int64_t r = 0; r < rows; ++r) {
    const int32_t *h = hist_ids ? hist_ids + hist_off[r] : NULL;
    int64_t hl = hist_ids ? hist_off[r + 1] - hist_off[r] : 0;
    int rc = orc_sample_row(logits + r * stride, vocab, h, hl, &cfgs[r], u[r],
                            method, &res[r],
                            cand_ids ? cand_ids + r * cap : NULL,
                            cand_vals ? cand_vals + r * cap : NULL,
                            cand_probs ? cand_probs + r * cap : NULL, cap);
    if (rc) return rc;
  }
  return 0;
}

/* src/kernels.ts:1616-1654, invocation by invocation.  `-1e30` is a WGSL
 * abstract float converted to f32 (src/kernels.ts:1629). */
void orc_wgsl_argmax(const float *logits, int64_t rows, int64_t stride, int64_t vocab,
                     int32_t *tokens) {
  enum { WG = 256 };
  float smax[WG];
  uint32_t sidx[WG];
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = logits + r * stride;
    for (uint32_t tid = 0; tid < WG; ++tid) {   /* src/kernels.ts:1628-1640 */
      float best_val = (float)-1e30;
      uint32_t best_idx = 0;
      for (int64_t i = tid; i < vocab; i += WG) {
        const float v = row[i];
        if (v > best_val) {
          best_val = v;
          best_idx = (uint32_t)i;
        }
      }
      smax[tid] = best_val;
      sidx[tid] = best_idx;
    }
    for (uint32_t s = WG / 2; s > 0; s >>= 1) {   /* src/kernels.ts:1641-1649 */
      for (uint32_t tid = 0; tid < s; ++tid) {
        if (smax[tid + s] > smax[tid]) {
          smax[tid] = smax[tid + s];
          sidx[tid] = sidx[tid + s];
        }
      }
    }
    tokens[r] = (int32_t)sidx[0];   /* src/kernels.ts:1650-1652 */
  }
}

/* src/wasm-backend.ts:1204-1215: the Wasm backend's greedy route.  bestVal
 * starts at the binary64 -1e30 and each logit (read exactly from its
 * Float32Array) replaces it only when strictly larger. */
void orc_wasm_greedy(const float *logits, int64_t rows, int64_t stride, int64_t vocab,
                     int32_t *tokens) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = logits + r * stride;
    double best_val = -1e30;
    int32_t best_idx = 0;
    for (int64_t i = 0; i < vocab; ++i) {
      const double v = (double)row[i];
      if (v > best_val) {
        best_val = v;
        best_idx = (int32_t)i;
      }
    }
    tokens[r] = best_idx;
  }
}
