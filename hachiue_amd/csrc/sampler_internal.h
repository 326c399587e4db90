// Internal definitions shared by the gfx950 sampler kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hs {

// Workgroup geometry of the row-chunk kernel: 256 threads (4 wave64s); each
// thread holds NV float4s, so one workgroup owns CHUNK consecutive logits of a
// row and each wave a contiguous quarter of it.
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kNV = 16;                        // float4 per thread
constexpr int kChunk = kThreads * kNV * 4;     // 16384 logits per workgroup
constexpr int kWaveSpan = kChunk / kWaves;     // 4096 logits per wave

// Candidate capacity per chunk (two layouts share it): the k<=64 path writes
// one list per wave at offsets w*kWaveCap; the k<=1024 path writes one list.
constexpr int kChunkCap = 2048;
constexpr int kWaveCap = kChunkCap / kWaves;   // 512
constexpr int kSmallK = 64;                    // wave-select path
constexpr int kMaxK = 1024;                    // largest k of the select paths
constexpr int kFinalCap = 12288;               // finalize LDS entries (>= X_row)

enum RowMode : int32_t {
  kModeGreedy = 0,   // temperature <= 0 (src/sampler.ts:36-46)
  kModeSmall = 1,    // 1 <= k <= 64
  kModeGeneric = 2,  // 64 < k <= 1024
  kModeLarge = 3,    // k > 1024 (nucleus over most of the row)
};

enum RowPen : int32_t {
  kPenRep = 1,       // repetition penalty active
  kPenPF = 2,        // presence / frequency extension active
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

// Per (row, chunk) summary written by the chunk kernel.
struct ChunkInfo {
  unsigned long long best;  // greedy: (key << 32) | ~index, 0 = none
  uint32_t thr;             // lower bound key all chunk candidates satisfy
  int32_t finite;           // finite logits in the chunk, -1 if not counted
  int32_t overflow;         // candidate lists truncated
  int32_t pad;
};
static_assert(sizeof(ChunkInfo) == 24, "ChunkInfo layout");

// Large-k path: per-chunk histogram of probability mass over key buckets
// below the row maximum.
constexpr int kLargeBuckets = 512;
constexpr int kLargeShift = 20;

struct Workspace {
  RowPlan *plans;            // [rows]
  uint2 *cand;               // [rows][S][kChunkCap] (key, index)
  int32_t *cand_count;       // [rows][S][kWaves]
  ChunkInfo *info;           // [rows][S]
};

struct LaunchArgs {
  float *logits;
  int64_t stride;
  int32_t rows;
  int32_t vocab;
  int32_t chunks;            // S = ceil(vocab / kChunk)
  int32_t vec;               // float4 loads allowed (alignment)
  int32_t any_pf;            // some row uses presence / frequency
  int32_t want_cands;        // exact candidate order must be produced
  const int32_t *hist_ids;
  const int64_t *hist_off;
  const double *uniforms;
  int32_t *tokens;
  int32_t cand_stride;
  int32_t *cand_ids;
  float *cand_probs;
  int32_t *cand_count_out;
  int32_t *cutoff_out;
  uint32_t *row_flags;
};

// Launches the two kernels on `stream`.  When `ev` is not null, records
// ev[0] before the chunk kernel, ev[1] between the kernels, ev[2] after.
constexpr int kTimedKernels = 2;
hipError_t launch_sample(const LaunchArgs &a, const Workspace &ws, hipStream_t stream,
                         hipEvent_t *ev);
hipError_t prepare_kernels();   // per device, once: raise dynamic LDS limits
size_t finalize_smem_bytes();

}  // namespace hs
