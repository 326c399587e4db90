/*
 * CPU restatement of hachiue's logits-to-token sampler (src/sampler.ts:1-118).
 *
 * TEST INFRASTRUCTURE ONLY.  This file and sampler_oracle.c are the checker
 * that the HIP sampler is compared against.  Only tests, the smoke check and
 * the CPU-baseline leg of the benchmark may load them; the product library
 * never links or calls this code.
 *
 * Arithmetic follows the reference exactly: logits are binary32 values, every
 * computation is binary64 (JavaScript numbers) and results are rounded to
 * binary32 only where the reference stores them into a Float32Array.
 */
#ifndef HACHIUE_SAMPLER_ORACLE_H
#define HACHIUE_SAMPLER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SampleConfig (src/sampler.ts:1-7) with every `??` default already resolved
 * (src/sampler.ts:18-22), plus the two penalties this build adds. */
typedef struct orc_config {
  double temperature;
  double top_k;              /* a JS number: Infinity, NaN and fractions allowed */
  double top_p;
  double min_p;
  double repetition_penalty;
  double presence_penalty;   /* extension, not in the reference */
  double frequency_penalty;  /* extension, not in the reference */
} orc_config;

enum {
  ORC_TOPK_LITERAL = 0, /* the reference's O(V*k) replace-min rescan, verbatim */
  ORC_TOPK_HEAP = 1     /* same slot semantics, first-minimum slot kept in a heap */
};

typedef struct orc_result {
  int32_t token;
  int32_t path;         /* 0 greedy, 1 no candidate, 2 single candidate, 3 drawn */
  int32_t k;            /* resolved slot count (src/sampler.ts:49) */
  int32_t n;            /* candidates after the sort (order.length) */
  int32_t cutoff;       /* kept prefix length after min-p / top-p */
  int32_t draw_index;   /* position in the sorted order the draw returned */
  double sum_prob;      /* unrounded binary64 sum of exp terms */
  double kept_sum;
  double draw_margin;   /* min_i |u*keptSum - cum_i| over the kept prefix */
  double topp_margin;   /* min_i |cum_i - topP| over the scanned prefix */
} orc_result;

/* Resolved slot count k = max(1, min(topK > 0 ? topK : 64, vocab)), truncated
 * the way `new Int32Array(k)` truncates its length.  Returns 1..vocab (or 1). */
int64_t orc_resolve_k(double top_k, int64_t vocab);

/* Repetition penalty (src/sampler.ts:24-33) followed by the presence /
 * frequency extension, in place. */
void orc_apply_penalties(float *logits, int64_t vocab, const int32_t *hist,
                         int64_t hist_len, const orc_config *cfg);

/* One call of sampleLogits on one row.  `logits` is mutated in place exactly as
 * the reference mutates its Float32Array.  `u` replaces Math.random().
 * Optional outputs (may be NULL): the first `cap` sorted candidates' ids,
 * values and normalised probabilities.  Returns 0, or -1 on allocation
 * failure. */
int orc_sample_row(float *logits, int64_t vocab, const int32_t *hist,
                   int64_t hist_len, const orc_config *cfg, double u,
                   int method, orc_result *res, int32_t *cand_ids,
                   float *cand_vals, float *cand_probs, int64_t cap);

/* Batch convenience: rows are independent, row r uses logits + r*stride,
 * history hist_ids[hist_off[r] .. hist_off[r+1]), cfgs[r] and u[r]. */
int orc_sample_batch(float *logits, int64_t rows, int64_t stride, int64_t vocab,
                     const int32_t *hist_ids, const int64_t *hist_off,
                     const orc_config *cfgs, const double *u, int method,
                     orc_result *res, int32_t *cand_ids, float *cand_vals,
                     float *cand_probs, int64_t cap);

/* The replace-min top-k scan alone (src/sampler.ts:48-69): final slot
 * contents.  Slots never filled keep id -1 / value -Infinity. */
int orc_topk_slots(const float *logits, int64_t vocab, int64_t k, int method,
                   int32_t *slot_ids, float *slot_vals);

/* The engine's GPU greedy route (src/engine.ts:1600-1601: temperature <= 0
 * and no repetition penalty) takes the WGSL argmax pipeline
 * (src/kernels.ts:1613-1654) instead of sampleLogits, simulated here step by
 * step: 256 invocations, invocation t scans ids t, t+256, ... with a strict
 * '>' from -1e30 (as binary32), then a shared-memory tree reduction with
 * stride 128, 64, ..., 1 in which slot t takes slot t+s only when strictly
 * greater.  Each row is `vocab` floats from logits + r*stride.  Writes one
 * id per row. */
void orc_wgsl_argmax(const float *logits, int64_t rows, int64_t stride, int64_t vocab,
                     int32_t *tokens);

/* src/wasm-backend.ts:1204-1215: the first id of the largest logit above the
 * binary64 -1e30 (strict '>'), 0 when none is; one id per row. */
void orc_wasm_greedy(const float *logits, int64_t rows, int64_t stride, int64_t vocab,
                     int32_t *tokens);

#ifdef __cplusplus
}
#endif

#endif
