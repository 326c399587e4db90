// Internal definitions shared by the gfx950 sampler kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hs {

// ---- row kernel: one 1024-thread workgroup streams a whole row: round 0 of
// 6 float4 per thread (24576 logits), then rounds of 8 float4 per thread
// (32768 logits), two rounds in flight at a time.
constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kR0NV = 6;                         // float4 per thread in round 0
constexpr int kR0F4 = kRowThreads * kR0NV;       // float4 of round 0
constexpr int kRowNV = 8;                        // float4 per thread per later round
constexpr int kRoundF4 = kRowThreads * kRowNV;   // float4 per later round
constexpr int kRowCandCap = 4096;                // streamed candidates per row
constexpr int kSegCap = kRowCandCap / kRowWaves; // of them per wave (its own segment)
constexpr int kRowMaxVocab = 1 << 19;            // LDS bitmap limit (64 KiB)
// Small batches split each row over kSplitMax workgroups at most (parts of at
// least kSplitMinPart logits), so that the batch fills the GPU's CUs.
constexpr int kSplitMax = 16;
constexpr int kSplitMinPart = 16384;
constexpr int kSplitCUs = 256;                   // workgroups a split call aims at
constexpr int kPartCap = 64;                     // candidates a part hands over (its top 64)

// ---- mid kernel (64 < k <= 1024): the row kernel's stream with a key
// histogram of kMidBins bins (the top 13 key bits: 1/16 octave) for the bound.
constexpr int kMidShift = 19;
constexpr int kMidBins = 1 << (32 - kMidShift);

// ---- chunk kernel: 256 threads own CHUNK consecutive logits of a row.
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kNV = 16;                          // float4 per thread
constexpr int kChunk = kThreads * kNV * 4;       // 16384 logits per workgroup
constexpr int kWaveSpan = kChunk / kWaves;       // 4096 logits per wave
constexpr int kChunkCap = 2048;                  // candidates per chunk (row region S*cap)

// ---- pen_kernel: one workgroup per row, an LDS hash table of the history's
// distinct ids.
constexpr int kPenThreads = 1024;
constexpr int kPenBits = 13;
constexpr int kPenSlots = 1 << kPenBits;         // table slots (64 KiB with the counts)
constexpr int kPenProbe = 64;                    // probes per insert before the range fallback
constexpr int kPenRange = 16384;                 // ids per range of the fallback
constexpr int kMidEarly = 2048;                  // mid kernel: a presence / frequency row's
                                                 //   listed (deferred) penalised ids
constexpr int kMidLdsMax = 152 * 1024;           // mid kernel: dynamic LDS ceiling

constexpr int kSmallK = 64;                      // wave-select paths
constexpr int kMaxK = 1024;                      // largest k of the select paths
constexpr int kFinalCap = 12288;                 // finalize: candidates >= X_row in LDS
constexpr int kSortCap = 2048;                   // candidates >= T sorted in LDS

enum RowMode : int32_t {
  kModeGreedy = 0,   // temperature <= 0 (src/sampler.ts:36-46)
  kModeSmall = 1,    // 1 <= k <= 64
  kModeGeneric = 2,  // 64 < k <= 1024
  kModeLarge = 3,    // k > 1024 (large_kernel)
};

enum RowPen : int32_t {
  kPenRep = 1,       // repetition penalty active
  kPenPF = 2,        // presence / frequency extension active (pre-pass applies all)
};

// Host-resolved per-row sampling plan (64 bytes).
struct RowPlan {
  double temperature;
  double top_p;
  double min_p;
  double rep;
  double pres;
  double freq;
  int32_t k;         // resolved slot count (src/sampler.ts:49)
  int32_t mode;      // RowMode
  int32_t pen;       // RowPen bits
  int32_t pad;
};
static_assert(sizeof(RowPlan) == 64, "RowPlan layout");

// Per (list position, chunk) summary written by the chunk kernel.
struct ChunkInfo {
  unsigned long long best;  // greedy: (key << 32) | ~index, 0 = none
  uint32_t thr;             // lower bound key all chunk candidates satisfy
  int32_t finite;           // finite logits in the chunk, -1 if not counted
  int32_t overflow;         // candidate list truncated
  int32_t pad;
};
static_assert(sizeof(ChunkInfo) == 24, "ChunkInfo layout");

// What a part of a split row hands over to the part that completes the row.
struct SplitMeta {
  unsigned long long best;   // greedy: packed maximum (global index), 0 = none
  int32_t count;             // candidates in the part's list, -1: overflowed
  uint32_t theta;            // their lower bound (a bound of the row's k-th largest)
  uint32_t key64;            // key of the part's 65th largest candidate (0: none)
  uint32_t pad;
};
static_assert(sizeof(SplitMeta) == 24, "SplitMeta layout");

// What a large-k row leaves for the slot replays when equal values make
// its order depend on the reference's slot history (k < the finite count).
struct ReplayReq {
  int32_t need;              // bit 0: the token; bit 1: the candidate ids;
                             //   bit 2 (kReplayDev): slots in device memory
  uint32_t xkey;             // the drawn value's key
  int32_t pos;               // the drawn position (value descending)
  int32_t mo;                // candidate positions to write
  uint32_t ckey;             // key at candidate position mo - 1
  int32_t pad;
};
static_assert(sizeof(ReplayReq) == 24, "ReplayReq layout");
constexpr int kReplayMaxK = 16384;     // slots the LDS replay holds
constexpr int kReplayCands = 1024;     // candidate positions it can order
// The replay with its slots in device memory (large_replay_dev_kernel): any
// k up to kReplayDevMaxK, kReplayDevCands candidate positions, at most
// kReplayDevBlocks workgroups, each with its own region of vocab keys, vocab
// ids and ceil(vocab / 64) first-level minima in the workspace.
constexpr int kReplayDev = 4;
constexpr int kReplayDevMaxK = 1 << 24;
constexpr int kReplayDevCands = 8192;
constexpr int kReplayDevBlocks = 16;

struct Workspace {
  RowPlan *plans;            // [rows]
  const int32_t *pf_list;    // rows penalised by the pre-pass
  const int32_t *row_list;   // rows of the row kernel
  const int32_t *chunk_list; // rows of the chunk + finalize kernels
  const int32_t *large_list; // rows of the large-k kernel
  const int32_t *mid_list;   // rows of the mid kernel
  const int32_t *lfast_list; // rows of the two-pass large-k kernel (k = vocab, no min-p)
  int32_t *large_retry;      // [n_lfast] 1: the two-pass kernel handed the row back
  ReplayReq *large_replay;   // [n_large] slot-history replays asked for by large_row
  uint32_t *replay_keys;     // [replay_dev][vocab] slots of the device-memory replay
  int32_t *replay_ids;       // [replay_dev][vocab]
  unsigned long long *replay_lvl1;  // [replay_dev][ceil(vocab / 64)] minima of 64 slots
  uint2 *cand;               // [n_chunk][S][kChunkCap] (key, index)
  int32_t *cand_count;       // [n_chunk]
  ChunkInfo *info;           // [n_chunk][S]
  unsigned long long *split_list;   // [n_row][split][kPartCap] packed candidates
  SplitMeta *split_meta;            // [n_row][split]
  uint32_t *split_cnt;              // [n_row] parts arrived (0 between calls)
};

struct LaunchArgs {
  float *logits;
  int64_t stride;
  int32_t rows;
  int32_t vocab;
  int32_t chunks;            // S = ceil(vocab / kChunk)
  int32_t vec;               // float4 loads allowed (alignment)
  int32_t want_cands;        // exact candidate order must be produced
  int32_t rows_direct;       // the row kernel takes every row: row = block index
  int32_t n_pf, n_row, n_chunk, n_large, n_mid;
  int32_t n_lfast;           // rows of the two-pass large-k kernel
  int32_t n_argmax;          // rows of the GPU greedy route (a call of its own)
  int32_t split;             // row / argmax kernel: workgroups per row (1: whole rows)
  int32_t replay_dev;        // workgroups of the device-memory slot replay (0: not launched)
  const int32_t *hist_ids;
  const int64_t *hist_off;   // packed lists: row r is hist_ids[off[r], off[r+1])
  const int64_t *hist_len;   // rings (hist_cap > 0): row r is hist_ids[r * cap, +cap),
  int64_t hist_cap;          //   len[r] ids appended so far, the last min(len, cap) kept
  // a decode step: where a row's token is written, its stop check and the
  // append to its ring (the writable hist_ids) happen too; null otherwise
  int32_t *dec_ring;
  int64_t *dec_len;
  int32_t *dec_done;
  const int32_t *dec_stop;
  int32_t dec_nstop;
  const double *uniforms;
  int32_t *tokens;
  int32_t cand_stride;
  int32_t *cand_ids;
  float *cand_probs;
  int32_t *cand_count_out;
  int32_t *cutoff_out;
  uint32_t *row_flags;
};

// Launches the kernels of one call on `stream`.  When `ev` is not null,
// ev[2i] and ev[2i + 1] receive the start and end of kernel i's dispatch
// (0 penalty pre-pass, 1 row kernel, 2 chunk kernel, 3 finalize, 4 large-k
// kernel, 5 mid kernel, 6 GPU greedy-route argmax, 8 two-pass large-k kernel,
// 9 the large-k slot replay, 10 the device-memory slot replay;
// 7 is the lm_head GEMV, launched apart), for the kernels that launch only:
// launched_kernels() says which.  The large-k kernel launches whenever a row
// has k > 1024: it also takes the rows the two-pass kernel hands back.
constexpr int kTimedKernels = 11;
inline unsigned launched_kernels(const LaunchArgs &a) {
  return (a.n_pf > 0 ? 1u : 0u) | (a.n_row > 0 ? 2u : 0u) | (a.n_chunk > 0 ? 12u : 0u) |
         (a.n_large + a.n_lfast > 0 ? 16u : 0u) | (a.n_mid > 0 ? 32u : 0u) |
         (a.n_argmax > 0 ? 64u : 0u) | (a.n_lfast > 0 ? 256u : 0u) | (a.n_large > 0 ? 512u : 0u) |
         (a.n_large > 0 && a.replay_dev > 0 ? 1024u : 0u);
}
// Largest vocabulary of the GPU greedy route (byte offsets of a row stay
// below 2^31).
constexpr int kArgmaxMaxVocab = 1 << 28;

// ---- lm_head GEMV (lmhead_kernels.hip)
// GGML type ids of the weight formats (src/types.ts:4-15).
constexpr int kW_F32 = 0, kW_Q4_0 = 2, kW_Q4_1 = 3, kW_Q4_K = 12, kW_Q6_K = 14;
// 128-weight binary / ternary formats, planar (quants and binary16 scales
// in two tensors, src/engine.ts:80-175): quant bytes per block
constexpr int kW_Q1_0 = 41, kW_PQ2_0 = 142, kW_PTQ1_0 = 143;
constexpr int tern_quant_bytes(int type) {
  return type == kW_Q1_0 ? 16 : type == kW_PQ2_0 ? 32 : type == kW_PTQ1_0 ? 26 : 0;
}
constexpr int kGemvThreads = 256;
constexpr int kGemvMaxK = 4096;       // x slices live in registers
constexpr int kGemvTimedSlot = 7;     // its start/end events in a timed call
struct GemvArgs {
  const float *x;            // [M][ldx]
  int64_t ldx;
  const void *w;             // N rows of row_bytes, GGML blocks
  uint32_t w_bytes, row_bytes;
  float *y;                  // [M][ldy]
  int64_t ldy;
  int32_t N, K, M, type;
  int32_t units;             // lane units per row
  int32_t seg;               // lanes per row (power of two, <= 64) when nru == 1
  int32_t nru;               // units per lane: 1, or 2 (a row takes all 64 lanes)
  int32_t blocks;            // workgroups per activation row
  // Q6_K: per activation row, part_cap slots of 16 partial sums and tile
  // counters (zero between calls) for the tiles cut between waves
  float *part;
  uint32_t *tile_cnt;
  int32_t part_cap;          // at least the waves of one activation row
  // Q1_0 / PQ2_0 / PTQ1_0: w holds the planar quants, scales the binary16
  // block scales (N * K / 128 of each), s_bytes their size
  const void *scales;
  uint32_t s_bytes;
};
// The 512-wide Hadamard rotation of a hadamard-folded weight's input
// (src/kernels.ts:177-227, mode 0): out[m][k] for m < M, k < K (K a multiple
// of 512), from x [M][ldx] and optional +-1 signs [K].
hipError_t launch_hadamard(const float *x, int64_t ldx, const float *signs, float *out, int M,
                           int K, hipStream_t stream);
constexpr int kGemvWavesPerCU = 16;   // Q4_K, Q6_K: the part_cap a CU needs
// Block formats go through LDS in batches of row steps (a step: the rows of
// one wave pass, 64 units): steps per batch and 16-byte reads per lane that
// hold a batch (its bytes plus the alignment of its start).
constexpr int gemv_batch_steps(int) { return 4; }
constexpr int gemv_unit_bytes2(int type) {   // twice a unit's bytes
  return type == kW_Q4_1 ? 40 : 36;
}
constexpr int gemv_batch_chunks(int type) {
  return (gemv_batch_steps(type) * 32 * gemv_unit_bytes2(type) + 32 + 1023) / 1024;
}
constexpr int gemv_lds_bytes(int type) { return (kGemvThreads / 64) * gemv_batch_chunks(type) * 1024; }
hipError_t launch_gemv(const GemvArgs &g, hipStream_t stream, hipEvent_t *ev, hipEvent_t done);
hipError_t prepare_gemv();      // per device, once (called by prepare_kernels)

// ---- decode step bookkeeping (after the sampler, same stream)
struct DecodeArgs {
  int32_t *tokens;           // [rows] the sampled tokens; -1 written for rows already done
  int32_t *ring;             // [rows][cap] history rings
  int64_t cap;
  int64_t *len;              // [rows] ids appended so far
  int32_t *done;             // [rows] 0 while generating, 1 once a stop token was drawn
  const int32_t *stop_ids;   // [n_stop]
  int32_t n_stop;
  int32_t rows;
};
constexpr int kMaxStopIds = 1024;
hipError_t launch_decode_append(const DecodeArgs &d, hipStream_t stream);
hipError_t launch_fill_u32(uint32_t *p, int64_t n, uint32_t v, hipStream_t stream);
hipError_t launch_gather_out(const float *src, const int64_t *idx, float *dst, int64_t n,
                             const int32_t *tok, int32_t *tok_dst, int32_t rows,
                             hipStream_t stream);
// `done`, when not null and `ev` is null, is recorded at the end of the
// call's last kernel (hipExtLaunchKernelGGL's stop event: no marker packet).
hipError_t launch_sample(const LaunchArgs &a, const Workspace &ws, hipStream_t stream,
                         hipEvent_t *ev, hipEvent_t done);
hipError_t prepare_kernels();   // per device, once: raise dynamic LDS limits
size_t row_smem_bytes(int vocab);
size_t mid_smem_bytes(int vocab);

// ---- the planar lm_head GEMV that samples its own rows (one launch)
// Workgroups of `kernel` resident at once on the current GPU (cached).
int resident_blocks(const void *kernel, uint32_t lds, int threads);
// Per activation row, zero between calls (the workgroup that completes the
// row resets it).
struct FuseRow {
  unsigned long long best;   // greedy: packed maximum of the row
  uint32_t arrived;          // workgroups done
  uint32_t pad;
};
static_assert(sizeof(FuseRow) == 16, "FuseRow layout");
constexpr int kFuseTiles = 8;     // 16-row tiles a wave of the fused GEMV records
constexpr int kFuseStage = 1024;  // entries the last workgroup ranks
constexpr int kFuseHist = 4096;   // bins of a row's key histogram (the keys' top 12 bits)
constexpr int kFuseWavesPerThread = 8;   // waves' entries a thread of the last workgroup reads
// Per wave of a row: the tiles it recorded, [0] their count, [1 + e] tile
// e (rows tile * 16 .. tile * 16 + 15).
constexpr int kFuseTileWords = 16;
static_assert(kFuseTileWords >= kFuseTiles + 1, "a wave's tiles fit");
struct FuseArgs {
  const RowPlan *plans;      // [M]: greedy or k <= 64, repetition penalty only
  const int32_t *hist_ids;   // packed lists (hist_off[m], hist_off[m + 1]) or null
  const int64_t *hist_off;
  const double *uniforms;    // [M]
  int32_t *tokens;           // [M]
  FuseRow *rows;             // [M]
  unsigned long long *wtop;  // [M][2][Bw]: each wave's largest, then its second largest
                             //   packed candidate (Bw = blocks * waves per workgroup)
  int32_t *wtiles;           // [M][Bw][kFuseTileWords] the tiles each wave recorded
  uint32_t *hist;            // [M][kFuseHist] workgroup maxima by key bin, zero between calls
  int32_t blocks;            // workgroups per activation row
};
hipError_t launch_tern_sample(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                              hipEvent_t *ev, hipEvent_t done);
// Every row greedy (any weight type): the GEMV keeps each workgroup's packed
// maximum, the last one writes the token (no candidate lists: f.wtop,
// f.wtiles, f.hist, f.blocks unused).
hipError_t launch_argmax_fused(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                               hipEvent_t *ev, hipEvent_t done);
int argmax_fused_grid(const GemvArgs &g);
// Its workgroups per activation row, or 0 when N needs more tiles per wave
// than it records (then the two-launch path is used).
int tern_sample_grid(const GemvArgs &g);
// Waves per workgroup of the one-launch kernel for lm_head weights of `type`.
int fuse_waves_per_block(int type);
// The same one launch for Q4_K and Q6_K lm_heads (greedy rows included), and
// its grid.
hipError_t launch_kq_sample(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                            hipEvent_t *ev, hipEvent_t done);
int kq_sample_grid(const GemvArgs &g);

}  // namespace hs
