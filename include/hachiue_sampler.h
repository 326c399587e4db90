/*
 * hachiue_sampler.h - C ABI of the MI355X (gfx950) logits-to-token sampler.
 *
 * Drop-in replacement for hachiue's CPU sampler `sampleLogits`
 * (src/sampler.ts:12-118, exported at src/index.ts:15).  The library runs the
 * whole sampling step on the GPU: repetition penalty over the last 128
 * history tokens (plus optional presence / frequency penalties), greedy
 * argmax, replace-min top-k with the reference's exact tie semantics, stable
 * sort, temperature softmax, min-p / top-p cutoff and the categorical draw.
 *
 * Conventions
 *  - Every entry point returns an hs_status; on failure hs_last_error() holds
 *    a message for the calling thread.  No C++ exception crosses the ABI.
 *  - Logits are mutated in place by the penalties, exactly as the reference
 *    mutates its Float32Array (src/sampler.ts:30).
 *  - A context owns one device, a workspace and the staging buffers.  Every
 *    entry point holds the context's lock for the whole call, so calls from
 *    several threads on one context run one after the other.  Device entry
 *    points enqueue work and return; a call on another stream than the
 *    previous call's first makes its stream wait for that call's last kernel
 *    (the workspace is shared), so streams may change between calls.
 *  - "device pointer" arguments must be device memory on the context's device
 *    (hipMalloc); "stream" is a hipStream_t or NULL for the null stream.
 */
#ifndef HACHIUE_SAMPLER_H
#define HACHIUE_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HS_ABI_VERSION 1

typedef enum hs_status {
  HS_OK = 0,
  HS_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, bad stride */
  HS_ERR_HIP = 2,              /* a HIP runtime call failed */
  HS_ERR_OUT_OF_MEMORY = 3,    /* workspace allocation failed */
  HS_ERR_UNSUPPORTED = 4       /* input outside what this build handles */
} hs_status;

/* SampleConfig (src/sampler.ts:1-7) after the `??` defaults of
 * src/sampler.ts:18-22 are resolved by the host layer.  Fields keep the
 * JavaScript-number meaning: top_k may be Infinity, NaN or fractional
 * (k = max(1, min(top_k > 0 ? top_k : 64, vocab)), truncated). */
typedef struct hs_sample_config {
  double temperature;        /* <= 0: greedy argmax (src/sampler.ts:36) */
  double top_k;
  double top_p;
  double min_p;
  double repetition_penalty; /* != 1: last 128 distinct ids (src/sampler.ts:25-33) */
  double presence_penalty;   /* extension; no reference counterpart */
  double frequency_penalty;  /* extension; no reference counterpart */
} hs_sample_config;

/* Per-row diagnostic bits written to row_flags (optional output). */
#define HS_ROW_GREEDY       0x1u /* temperature <= 0 path */
#define HS_ROW_REPLAYED     0x2u /* exact replace-min replay was needed (ties) */
#define HS_ROW_TIES         0x4u /* equal values among or at the candidates */
#define HS_ROW_SINGLE       0x8u /* 0 or 1 candidate: no draw consumed */
#define HS_ROW_UNSUPPORTED 0x10u /* top-k > 16777216 (a vocab above that) below
                                    the finite count with a group of equal values
                                    at the drawn position: the reference orders it
                                    by its slot history, which this build replays
                                    for top-k up to 16777216; token is -1.  Also set
                                    (token kept) when candidate outputs would need
                                    more than 8192 slot-ordered positions or more
                                    than 2048 positions above the last listed
                                    value on the top-k > 1024 path */
#define HS_ROW_LARGE       0x20u /* top-k > 1024 path: binary64 sums in another order
                                    than the reference's (probabilities within 1e-5) */
#define HS_ROW_TWO_PASS    0x40u /* with HS_ROW_LARGE: a top-k = vocab row finished by
                                    the two-pass kernel (bucketed probability mass,
                                    exact walk of the buckets at the cutoff and draw) */

typedef struct hs_context hs_context;

/* Library identity. */
int hs_abi_version(void);
const char *hs_last_error(void);

/* Reference defaults of src/sampler.ts:18-22 (temperature 0.6, topK 20,
 * topP 0.95, minP 0, repetitionPenalty 1) and 0 for the extensions. */
void hs_config_default(hs_sample_config *config);

/* Context on HIP device `device`.  Allocates the workspace lazily and grows it
 * when a call needs more; a call that fits the current workspace allocates
 * nothing. */
int hs_context_create(int device, hs_context **out);
int hs_context_destroy(hs_context *ctx);

/* Drop-in for sampleLogits(logits, vocab, history, config)
 * (src/sampler.ts:12-17) on one HOST row.  `logits` (at least vocab floats)
 * is updated in place with the penalised values; `uniform` in [0, 1) replaces
 * Math.random() (src/sampler.ts:112) and is consumed only when a draw
 * happens.  Blocks until *token_out is written. */
int hs_sample_logits(hs_context *ctx, float *logits, int32_t vocab,
                     const int32_t *history, int64_t history_len,
                     const hs_sample_config *config, double uniform,
                     int32_t *token_out);

/* Batched host variant: `rows` rows of `row_stride` floats; row r's history
 * is hist_ids[hist_offsets[r] .. hist_offsets[r+1]) (hist_offsets has rows+1
 * entries; both may be NULL for no history); configs[r], uniforms[r].  Copies
 * in, samples, copies tokens and penalised logits back.  Blocks.
 * HS_ERR_UNSUPPORTED when a row ends with HS_ROW_UNSUPPORTED (see above). */
int hs_sample_logits_batch(hs_context *ctx, float *logits, int32_t rows,
                           int64_t row_stride, int32_t vocab,
                           const int32_t *hist_ids, const int64_t *hist_offsets,
                           const hs_sample_config *configs,
                           const double *uniforms, int32_t *tokens_out);

/* Device-resident batch, asynchronous on `stream`: d_logits, d_hist_ids,
 * d_hist_offsets, d_uniforms and d_tokens are device pointers; `configs` is a
 * HOST array of `rows` configs (staged to the device by the library, skipped
 * when identical to the previous call's).  Optional device outputs (each may
 * be NULL): the first `cand_stride` sorted candidates per row (ids, normalised
 * probabilities), the candidate count, the kept-prefix length and row flags.
 * A row with HS_ROW_UNSUPPORTED gets token -1. */
int hs_sample_batch_device(hs_context *ctx, float *d_logits, int32_t rows,
                           int64_t row_stride, int32_t vocab,
                           const int32_t *d_hist_ids,
                           const int64_t *d_hist_offsets,
                           const hs_sample_config *configs,
                           const double *d_uniforms, int32_t *d_tokens,
                           void *stream);

int hs_sample_batch_device_ex(hs_context *ctx, float *d_logits, int32_t rows,
                              int64_t row_stride, int32_t vocab,
                              const int32_t *d_hist_ids,
                              const int64_t *d_hist_offsets,
                              const hs_sample_config *configs,
                              const double *d_uniforms, int32_t *d_tokens,
                              int32_t cand_stride, int32_t *d_cand_ids,
                              float *d_cand_probs, int32_t *d_cand_count,
                              int32_t *d_cutoff, uint32_t *d_row_flags,
                              void *stream);

/* hs_sample_batch_device without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate during the call (tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, semantics
 * and outputs as hs_sample_batch_device; the workspace is one static device
 * array per GPU (about 4.5 MB: 350 KB of plans, lists and hand-over buffers
 * and one 4 MB region of the large-k slot replay; held until the process
 * ends, its address taken once per device when the first context on it is
 * created), and the plans are staged through pinned memory the context set
 * up at creation.  The call makes no hipMalloc, hipFree, host allocation or
 * hipMemset.  Limits: rows <= 2048 and vocab <= 524288 (HS_ERR_UNSUPPORTED
 * beyond).  It must not be captured into a HIP graph: it may wait for its
 * previous plan upload, and a replay would read plans that later calls have
 * rewritten (a call on a capturing stream returns HS_ERR_UNSUPPORTED).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU through different contexts race (calls on one context are serialised
 * as usual).  Kernel timing (hs_context_set_timing) does not cover this
 * entry point. */
int hs_sample_batch_device_noalloc(hs_context *ctx, float *d_logits, int32_t rows,
                                   int64_t row_stride, int32_t vocab,
                                   const int32_t *d_hist_ids,
                                   const int64_t *d_hist_offsets,
                                   const hs_sample_config *configs,
                                   const double *d_uniforms, int32_t *d_tokens,
                                   void *stream);

/* The engine's GPU greedy route.  hachiue's engine decodes greedily without
 * sampleLogits when temperature <= 0 and no repetition penalty is set
 * (src/engine.ts:1600-1601): the forward pass ends in the WGSL argmax
 * pipeline (src/kernels.ts:1613-1654, one 256-invocation workgroup per row,
 * output u32 outToken).  These entry points replace that pipeline with its
 * exact tie order, which differs from sampleLogits' greedy argmax
 * (src/sampler.ts:36-46) on equal maxima, NaN and values at or below
 * -1e30: invocation t keeps the first id of its maximum over ids t, t+256, ...
 * (strict '>' from f32(-1e30)) and the tree reduction keeps slot t against
 * slot t+s on a tie, so among equal maxima the id whose low byte, bit-reversed,
 * is smallest wins, then the smallest id; no value above f32(-1e30) gives 0.
 * Logits are read only.  `rows` rows of `row_stride` floats (the reference's
 * rowOffset * vocab addressing is row_stride == vocab); vocab up to 2^28.
 * hs_argmax_device is asynchronous on `stream` (device pointers);
 * hs_argmax copies host rows in and the ids out, and blocks. */
int hs_argmax_device(hs_context *ctx, const float *d_logits, int32_t rows,
                     int64_t row_stride, int32_t vocab, int32_t *d_tokens,
                     void *stream);
int hs_argmax(hs_context *ctx, const float *logits, int32_t rows,
              int64_t row_stride, int32_t vocab, int32_t *tokens_out);

/* The logits producer in front of the sampler: hachiue's lm_head GEMV
 * (src/engine.ts:1493-1515, runMatmul of output.weight; WGSL pipelines
 * gemv_f32 / gemv_q4_0 / gemv_q4_1 / gemv_q4_k / gemv_q6_k,
 * src/kernels.ts:244-290, :717-1090; the planar Q1_0 / PQ2_0 / PTQ1_0 and
 * Hadamard-folded weights go through hs_gemv_device_ex).
 * y[m][n] = sum_k x[m][k] W[n][k] for
 * m < M, n < N; x is [M][ldx] binary32, y is [M][ldy] binary32, W is the
 * GGUF tensor's raw blocks of `w_type` (GGML ids: 0 F32, 2 Q4_0, 3 Q4_1,
 * 12 Q4_K, 14 Q6_K), N rows of K weights back to back, as the reference
 * uploads them (src/engine.ts:772-800).  K a multiple of the block size,
 * K <= 4096, W at most 4 GiB and 16-byte aligned.  Results differ from the
 * reference's binary32 sums by rounding only.  Q4_K and Q6_K run on the
 * matrix cores with x held as integer limbs: a non-finite element of an x row
 * makes every result of that row NaN (the reference's binary32 sums give NaN
 * or +-Infinity there).  Asynchronous on `stream`. */
int hs_gemv_device(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx,
                   int32_t K, const void *d_w, int32_t w_type, int32_t N,
                   float *d_y, int64_t ldy, void *stream);

/* A weight tensor as the reference's GPU holds it (GpuTensor,
 * src/engine.ts:736-800): its GGML type, N rows of K weights, whether it
 * was folded with the 512-wide Hadamard rotation (hadamardFolded,
 * src/engine.ts:816-822), and its data:
 *   - F32, Q4_0, Q4_1, Q4_K, Q6_K: `data` holds the raw GGUF blocks, rows
 *     back to back, 16-byte aligned; `scales16` is NULL;
 *   - Q1_0 (41), PQ2_0 (142), PTQ1_0 (143), 128 weights per block: the
 *     planar form the reference uploads (src/engine.ts:80-175):
 *     `data` holds every block's quant bytes (16, 32 or 26 per block; rows
 *     of K / 128 blocks back to back; 16-byte aligned, PTQ1_0 4-byte),
 *     `scales16` the blocks' binary16 scales in the same order (4-byte
 *     aligned).  hs_split_blocks makes both from GGUF blocks.
 * With `hadamard` set, the GEMV's input is rotated first, as
 * src/engine.ts:1121-1145 does: each 512-block of x is multiplied by
 * `signs` (K floats of +-1, or NULL for none; arch.hadamard's sign vector of
 * width K), transformed by the Walsh-Hadamard butterflies and scaled by
 * binary32(1/sqrt(512)) (src/kernels.ts:177-227); K must be a multiple of
 * 512. */
typedef struct hs_weights {
  int32_t type;
  int32_t rows;            /* N */
  int32_t cols;            /* K */
  int32_t hadamard;        /* nonzero: hadamardFolded */
  const void *data;
  const void *scales16;
  const float *signs;
} hs_weights;

/* hs_gemv_device for any hs_weights (the only entry point for the planar
 * types and for Hadamard-folded weights).  Planar types: every result lies
 * within 2^-16 * sum_k |x_k w_k| of the exact product, like the others;
 * their kernel holds x as four 7-bit limbs relative to each 128-block's
 * largest |x|, so an element below about 2^-28 of that maximum counts as 0.
 * A non-finite element of an x row makes every result of that row NaN.
 * Asynchronous on `stream`; a folded weight's rotated input lives in the
 * context's workspace. */
int hs_gemv_device_ex(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx,
                      const hs_weights *w, float *d_y, int64_t ldy, void *stream);

/* GGUF blocks of Q1_0 ([binary16 d][16 B sign bits]), PQ2_0 ([d][32 B
 * codes]) or PTQ1_0 ([24 B qs][2 B qh][d]) into planar quants
 * (n_blocks * 16, 32 or 26 bytes) and binary16 scales (n_blocks * 2 bytes),
 * on the host: the byte split of the reference's upload
 * (src/engine.ts:80-175 createBlockSplitter). */
int hs_split_blocks(int32_t type, const void *blocks, int64_t n_blocks, void *quants,
                    void *scales16);

/* lm_head and sampler in one call on one stream, with no host round trip in
 * between (the reference reads the logits back to the host, src/engine.ts:
 * 1526-1531, and samples there): hs_gemv_device into d_logits ([M][ldl],
 * N = vocab), then hs_sample_batch_device over its M rows. */
int hs_lm_head_sample_device(hs_context *ctx, const float *d_x, int32_t M,
                             int64_t ldx, int32_t K, const void *d_w,
                             int32_t w_type, int32_t N, float *d_logits,
                             int64_t ldl, const int32_t *d_hist_ids,
                             const int64_t *d_hist_offsets,
                             const hs_sample_config *configs,
                             const double *d_uniforms, int32_t *d_tokens,
                             void *stream);

/* hs_lm_head_sample_device for any hs_weights (N = w->rows = vocab). */
int hs_lm_head_sample_device_ex(hs_context *ctx, const float *d_x, int32_t M,
                                int64_t ldx, const hs_weights *w, float *d_logits,
                                int64_t ldl, const int32_t *d_hist_ids,
                                const int64_t *d_hist_offsets,
                                const hs_sample_config *configs,
                                const double *d_uniforms, int32_t *d_tokens,
                                void *stream);

/* One step of the decode loop with the token history on the GPU
 * (src/engine.ts:1626-1644, whose tokenHistory is a host array, and whose
 * stopSet check, :1628, runs on the host after a readback of the token).
 * Per row r, on `stream`, without a host synchronisation:
 *   1. the token is drawn from d_logits as hs_sample_batch_device does, with
 *      row r's history read from its ring: d_ring[r * ring_cap, +ring_cap)
 *      holds the last min(d_len[r], ring_cap) ids appended, the id appended
 *      as the j-th (0-based) at slot j mod ring_cap;
 *   2. a row with d_done[r] != 0 (done before this step), or whose draw
 *      is left unresolved (HS_ROW_UNSUPPORTED), gets d_tokens[r] = -1 and
 *      keeps its state; a drawn id in
 *      d_stop_ids[0, n_stop) sets d_done[r] = 1 (the id is reported in
 *      d_tokens[r] and does not join the history); any other id is written
 *      to slot d_len[r] mod ring_cap and d_len[r] is incremented.
 * The repetition penalty reads the last 128 ids (ring_cap >= 128 keeps that
 * window exact); presence / frequency count the last min(len, ring_cap) ids,
 * the full history while ring_cap >= len.  The stop check and the append run
 * in the lane that writes the row's token, inside the sampler's kernels.  The caller fills the rings with
 * the prompt ids (d_len[r] = prompt length) before the first step, bounds
 * the steps (maxNewTokens, the sequence length) and reads d_done / d_tokens
 * when it wants to (src/engine.ts:1631, onToken).  Greedy rows
 * (temperature <= 0) take src/sampler.ts:36-46's first maximum, not the
 * WGSL argmax order of hs_argmax_device.  ring_cap in [128, 2^29], n_stop in
 * [0, 1024]; d_uniforms[r] as in hs_sample_batch_device (one set per step). */
int hs_decode_step_device(hs_context *ctx, float *d_logits, int32_t rows,
                          int64_t row_stride, int32_t vocab, int32_t *d_ring,
                          int64_t ring_cap, int64_t *d_len, int32_t *d_done,
                          const int32_t *d_stop_ids, int32_t n_stop,
                          const hs_sample_config *configs,
                          const double *d_uniforms, int32_t *d_tokens,
                          void *stream);

/* Diagnostics (no counterpart in the reference, which has no GPU sampler):
 * while enabled, every sampling call records HIP events on its stream around
 * each of its kernel launches.  hs_context_kernel_times() waits for the
 * recorded calls, writes the summed device milliseconds per kernel
 * (ms[0] presence/frequency pre-pass, ms[1] row kernel, ms[2] chunk kernel,
 * ms[3] finalize, ms[4] large-k kernel, ms[5] mid-k kernel, ms[6] greedy-route
 * argmax, ms[7] lm_head GEMV, ms[8] two-pass large-k kernel, ms[9] large-k
 * slot replay in LDS, ms[10] large-k slot replay in device memory; a kernel
 * a call did not launch adds 0)
 * and the number of
 * timed calls, and resets the totals. */
int hs_context_set_timing(hs_context *ctx, int enable);
int hs_context_kernel_times(hs_context *ctx, double *ms, int32_t count, int64_t *calls);

#ifdef __cplusplus
}
#endif

#endif
