// C ABI of the gfx950 sampler: contexts, workspace, per-row plans, argument
// validation and the host / device entry points declared in
// include/hachiue_sampler.h.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "hachiue_sampler.h"
#include "sampler_internal.h"

// ---- workspace of hs_sample_batch_device_noalloc: one array per GPU, in
// device memory for the life of the process.  Layout (offsets 256-aligned):
// plans [kMaxRows] | routing lists [5][kMaxRows] | the two-pass large-k
// rows handed back [kMaxRows] | slot-replay requests [kMaxRows] | split-row
// hand-over lists
// [kSplitCUs][kPartCap] | their meta data [kSplitCUs] | the split rows'
// arrival counters [kSplitCUs] (zero between calls) | one region of the
// device-memory slot replay: keys [kRowMaxVocab], ids [kRowMaxVocab], the
// minima of each 64 slots [kRowMaxVocab / 64].
namespace na {
constexpr int kMaxRows = 2048;
constexpr size_t kPlansOff = 0;
constexpr size_t kPlansBytes = sizeof(hs::RowPlan) * kMaxRows;
constexpr size_t kListsOff = kPlansOff + kPlansBytes;
constexpr size_t kListsBytes = sizeof(int32_t) * 5 * kMaxRows;
constexpr size_t kRetryOff = kListsOff + kListsBytes;
constexpr size_t kRetryBytes = sizeof(int32_t) * kMaxRows;
constexpr size_t kReplayOff = kRetryOff + kRetryBytes;
constexpr size_t kReplayBytes = sizeof(hs::ReplayReq) * kMaxRows;
constexpr size_t kSplitListOff = kReplayOff + kReplayBytes;
constexpr size_t kSplitListBytes = sizeof(unsigned long long) * hs::kSplitCUs * hs::kPartCap;
constexpr size_t kSplitMetaOff = kSplitListOff + kSplitListBytes;
constexpr size_t kSplitMetaBytes = sizeof(hs::SplitMeta) * hs::kSplitCUs;
constexpr size_t kSplitCntOff = kSplitMetaOff + kSplitMetaBytes;
constexpr size_t kSplitCntBytes = sizeof(uint32_t) * hs::kSplitCUs;
constexpr size_t kRKeysOff = (kSplitCntOff + kSplitCntBytes + 255) / 256 * 256;
constexpr size_t kRSlotBytes = sizeof(uint32_t) * hs::kRowMaxVocab;
constexpr size_t kRIdsOff = kRKeysOff + kRSlotBytes;
constexpr size_t kRLvl1Off = kRIdsOff + kRSlotBytes;
constexpr size_t kRLvl1Bytes = sizeof(unsigned long long) * (hs::kRowMaxVocab / 64);
constexpr size_t kBytes = kRLvl1Off + kRLvl1Bytes;
static_assert(kListsOff % 256 == 0 && kRetryOff % 256 == 0 && kReplayOff % 256 == 0 &&
                  kSplitListOff % 256 == 0 &&
                  kSplitMetaOff % 256 == 0 &&
                  kSplitCntOff % 256 == 0 && kRKeysOff % 256 == 0 && kRIdsOff % 256 == 0 &&
                  kRLvl1Off % 256 == 0,
              "scratch layout alignment");
constexpr int kMaxDevices = 64;
}  // namespace na

// In host code `scratch` names a host-side stand-in: kernels and copies take
// the per-device address from hipGetSymbolAddress (g_scratch below).
static __device__ __align__(256) unsigned char scratch[na::kBytes];

namespace {

thread_local std::string g_error;

int fail(int status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return status;
}

// Failure injection for tests of the error paths: with HS_INJECT_HIP_FAILURE=n
// in the environment when a context is created, the n-th HIP runtime call
// checked through HS_HIP after that (0: the first) is not made and reports
// hipErrorOutOfMemory instead; -1 (the default) injects nothing.
std::atomic<int> g_inject{-1};

bool inject_failure() {
  int v = g_inject.load(std::memory_order_relaxed);
  while (v >= 0) {
    if (g_inject.compare_exchange_weak(v, v - 1, std::memory_order_relaxed)) return v == 0;
  }
  return false;
}

#define HS_HIP(call)                                                                \
  do {                                                                              \
    hipError_t e_ = inject_failure() ? hipErrorOutOfMemory : (call);                \
    if (e_ != hipSuccess)                                                           \
      return fail(HS_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_));       \
  } while (0)

// Grow-only device buffer.
struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  hipError_t ensure(size_t need) {
    if (need <= bytes) return hipSuccess;
    if (p) {
      hipError_t e = hipDeviceSynchronize();   // no launch may still use it
      if (e != hipSuccess) return e;
      (void)hipFree(p);
      p = nullptr;
      bytes = 0;
    }
    size_t b = need + need / 4;
    hipError_t e = hipMalloc(&p, b);
    if (e != hipSuccess) { p = nullptr; return e; }
    bytes = b;
    return hipSuccess;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
};

// Grow-only pinned host buffer (hipHostMalloc: the device reads and writes it
// directly, and copies from it are truly asynchronous).
struct PinBuf {
  void *p = nullptr;
  size_t bytes = 0;
  hipError_t ensure(size_t need) {
    if (need <= bytes) return hipSuccess;
    if (p) {
      (void)hipHostFree(p);
      p = nullptr;
      bytes = 0;
    }
    size_t b = need + need / 4;
    hipError_t e = hipHostMalloc(&p, b);
    if (e != hipSuccess) { p = nullptr; return e; }
    bytes = b;
    return hipSuccess;
  }
  void release() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    bytes = 0;
  }
};

// Host entry points stage a logits block of at most this size through the
// context's pinned buffer (larger blocks are copied from the caller's memory
// directly).
constexpr size_t kPinLogitsMax = size_t(64) << 20;
// Up to this size, a host call whose rows all stream their logits once (no
// top-k above 1024) lets the kernels read the pinned staging directly and
// write the tokens and penalised logits back into it: no copy to device
// memory and none back.
constexpr size_t kZeroCopyMax = size_t(4) << 20;
constexpr size_t pin_align(size_t b) { return (b + 255) / 256 * 256; }

// Routing of rows to kernels, uploaded next to the plans.
struct Routing {
  std::vector<int32_t> pf, row, chunk, large, mid, lfast;
};

std::mutex g_prep_mu;
std::vector<int> g_prepared;
// per device: the address of `scratch` on that device (set once, at the
// first context created on it) and a count of the plan uploads into it
void *g_scratch[na::kMaxDevices];
std::atomic<uint64_t> g_scratch_gen[na::kMaxDevices];

}  // namespace

struct hs_context {
  int device = 0;
  // every entry point holds it for the whole call: calls on one context are
  // serialised (the workspace, staging and host buffers are shared)
  std::mutex mu;
  // recorded at the end of each call's last kernel on done_stream; a call on
  // another stream waits for it before it touches the workspace
  hipEvent_t done_ev = nullptr;
  hipStream_t done_stream = nullptr;
  bool has_done = false;
  // workspace
  DevBuf plans, cand, cand_count, info;
  DevBuf split_list, split_meta, split_cnt;   // split rows (split_cnt: zero between calls)
  DevBuf gemv_part, gemv_cnt;   // Q4_K/Q6_K GEMV tiles cut between waves (gemv_cnt: zero between calls)
  DevBuf gemv_rot;              // the Hadamard-rotated input of a folded weight
  DevBuf fuse_rows, fuse_pool, fuse_hist;   // lm_head GEMV that samples its rows: counters
                                //   (zero between calls), the waves' two largest, the
                                //   rows' key histograms (zero between calls)
  // HS_LMHEAD_FUSE at creation: 0 always two launches; 1 (default) one
  // launch for all-greedy calls on the planar, Q4_K and Q6_K weights; 2 also
  // for calls with k <= 64 sampling rows there and all-greedy calls on the
  // vector-unit weights (F32, Q4_0, Q4_1)
  int fuse = 1;
  DevBuf large_retry;           // two-pass large-k rows handed back
  DevBuf large_replay;          // slot-history replays asked for by the large-k kernel
  DevBuf replay_slots;          // the device-memory replay's regions: keys, then ids
  int64_t cand_count_rows = 0;     // rows whose counter is known to be zero
  // plan upload cache
  std::vector<hs::RowPlan> last_plans;
  std::vector<hs::RowPlan> call_plans;   // the current call's plans and routing
  Routing call_rt;                       //   (kept to reuse their storage)
  int last_vocab = -1;
  void *plan_staging = nullptr;          // pinned
  size_t plan_staging_bytes = 0;
  hipEvent_t plan_done = nullptr;
  bool plan_pending = false;
  // host entry points
  DevBuf h_logits, h_small, h_tok;  // logits block; uniforms | offsets | history ids
  PinBuf h_pin;                   // staging of the same, the penalised entries' offsets,
                                  //   and the outputs the device writes back
  std::vector<int64_t> gidx;      // offsets of the penalised entries in the logits block
  hipStream_t stream = nullptr;
  // per-kernel timing diagnostics
  bool timing = false;
  struct TimedCall {
    unsigned mask;                         // launched_kernels() of the call
    hipEvent_t ev[2 * hs::kTimedKernels];  // start/end per launched kernel
  };
  std::vector<hipEvent_t> ev_free;
  std::vector<TimedCall> timed;
  double kernel_ms[hs::kTimedKernels] = {};
  // rows routed to the row kernel only when a call has at least this many
  int row_min_rows = 1;
  // workgroups per row of the row kernel: 0 chooses by batch size
  int row_split = 0;
  int64_t timed_calls = 0;
  // hs_sample_batch_device_noalloc: pinned staging of plans and lists, the
  // configs of this context's last upload into the device's scratch, and the
  // device's upload count after it (all set up at creation)
  void *na_staging = nullptr;
  hipEvent_t na_upload_ev = nullptr;
  bool na_pending = false;
  hs_sample_config *na_last = nullptr;
  int na_rows = -1, na_vocab = -1;
  int na_count[6] = {0, 0, 0, 0, 0, 0};   // pf, row, large, mid, two-pass large; and
                                           //   whether a large row has k > kReplayMaxK
  uint64_t na_gen = 0;
};

namespace {

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// The workspace is shared by every call on a context: a call on another
// stream than the previous call's waits for that call's last kernel.
int enter_stream(hs_context *ctx, hipStream_t s) {
  if (ctx->has_done && s != ctx->done_stream) HS_HIP(hipStreamWaitEvent(s, ctx->done_ev, 0));
  return HS_OK;
}

// After a call's launches on `s`: `recorded` says whether done_ev was
// attached to its last kernel; otherwise it is recorded here.
int leave_stream(hs_context *ctx, hipStream_t s, bool recorded) {
  if (!recorded) HS_HIP(hipEventRecord(ctx->done_ev, s));
  ctx->done_stream = s;
  ctx->has_done = true;
  return HS_OK;
}

// src/sampler.ts:49 k = Math.max(1, Math.min(topK > 0 ? topK : 64, vocab)),
// truncated as `new Int32Array(k)` truncates a fractional length.
int64_t resolve_k(double top_k, int64_t vocab) {
  const double t = (top_k > 0) ? top_k : 64.0;
  const double m = t < (double)vocab ? t : (double)vocab;
  const double k = m > 1.0 ? m : 1.0;
  return (int64_t)floor(k);
}

// k = vocab (no slot is ever evicted) and no min-p: the two-pass large-k
// kernel's rows.
bool two_pass_large(const hs::RowPlan &p, int vocab) {
  return p.mode == hs::kModeLarge && p.k >= vocab && !(p.min_p > 0.0);
}

// One row's plan: the `??`-resolved config of src/sampler.ts:18-22 with k
// resolved (:49) and the kernel mode.
hs::RowPlan plan_row(const hs_sample_config &c, int vocab) {
  hs::RowPlan p;
  memset(&p, 0, sizeof p);
  p.temperature = c.temperature;
  p.top_p = c.top_p;
  p.min_p = c.min_p;
  p.rep = c.repetition_penalty;
  p.pres = c.presence_penalty;
  p.freq = c.frequency_penalty;
  p.pen = (c.repetition_penalty != 1.0 ? hs::kPenRep : 0) |
          ((c.presence_penalty != 0.0 || c.frequency_penalty != 0.0) ? hs::kPenPF : 0);
  if (c.temperature <= 0) {   // src/sampler.ts:36 (NaN is not <= 0)
    p.mode = hs::kModeGreedy;
    p.k = 1;
  } else {
    const int64_t k = resolve_k(c.top_k, vocab);
    p.k = (int32_t)k;
    if (k <= hs::kSmallK) p.mode = hs::kModeSmall;
    else if (k <= hs::kMaxK) p.mode = hs::kModeGeneric;
    else p.mode = hs::kModeLarge;
  }
  return p;
}

// The large-k kernel takes penalised logits: its rows' penalties run in the
// pre-pass, like the presence / frequency rows of the row and chunk kernels.
// The mid kernel applies its presence / frequency rows' penalties itself
// (`mid`: the row is routed to it).
bool in_prepass(const hs::RowPlan &p, bool mid) {
  return ((p.pen & hs::kPenPF) && !mid) || (p.pen && p.mode == hs::kModeLarge);
}

int build_plans(const hs_sample_config *cfgs, int rows, int vocab, int row_min_rows,
                std::vector<hs::RowPlan> &out, Routing &rt) {
  out.resize((size_t)rows);
  rt.pf.clear();
  rt.row.clear();
  rt.chunk.clear();
  rt.large.clear();
  rt.mid.clear();
  rt.lfast.clear();
  for (int r = 0; r < rows; ++r) {
    const hs::RowPlan p = plan_row(cfgs[r], vocab);
    out[(size_t)r] = p;
    if (p.mode == hs::kModeLarge) {
      (two_pass_large(p, vocab) ? rt.lfast : rt.large).push_back(r);
      continue;
    }
    const bool one_pass = vocab <= hs::kRowMaxVocab && rows >= row_min_rows;
    if (one_pass && p.mode == hs::kModeGeneric) rt.mid.push_back(r);
    else if (one_pass) rt.row.push_back(r);
    else rt.chunk.push_back(r);
  }
  // In a call that launches the mid kernel anyway, its rows with k <= 64 join
  // it: one launch over all of them instead of two in sequence, each filling
  // only part of the GPU.  Greedy rows stay with the row kernel.
  if (!rt.mid.empty() && !rt.row.empty()) {
    std::vector<int32_t> keep;
    for (int32_t r : rt.row) (out[(size_t)r].mode == hs::kModeSmall ? rt.mid : keep).push_back(r);
    rt.row.swap(keep);
  }
  std::vector<char> mid((size_t)rows, 0);
  for (int32_t r : rt.mid) mid[(size_t)r] = 1;
  for (int r = 0; r < rows; ++r)
    if (in_prepass(out[(size_t)r], mid[(size_t)r] != 0)) rt.pf.push_back(r);
  return HS_OK;
}

// Uploads plans and routing lists (skipped when identical to the last call's).
int upload_plans(hs_context *ctx, const std::vector<hs::RowPlan> &plans, const Routing &rt,
                 int vocab, hipStream_t stream) {
  const size_t rows = plans.size();
  const size_t pbytes = rows * sizeof(hs::RowPlan);
  const size_t lbytes =
      sizeof(int32_t) * (rt.pf.size() + rt.row.size() + rt.chunk.size() + rt.large.size() +
                         rt.mid.size() + rt.lfast.size());
  const size_t bytes = pbytes + lbytes;
  if (ctx->last_plans.size() == rows && ctx->last_vocab == vocab && ctx->plans.bytes >= bytes &&
      memcmp(ctx->last_plans.data(), plans.data(), pbytes) == 0)
    return HS_OK;
  HS_HIP(ctx->plans.ensure(bytes));
  if (ctx->plan_pending) {   // the staging buffer may still be read by a copy
    HS_HIP(hipEventSynchronize(ctx->plan_done));
    ctx->plan_pending = false;
  }
  if (ctx->plan_staging_bytes < bytes) {
    if (ctx->plan_staging) (void)hipHostFree(ctx->plan_staging);
    ctx->plan_staging = nullptr;
    ctx->plan_staging_bytes = 0;
    HS_HIP(hipHostMalloc(&ctx->plan_staging, bytes));
    ctx->plan_staging_bytes = bytes;
  }
  char *st = static_cast<char *>(ctx->plan_staging);
  memcpy(st, plans.data(), pbytes);
  int32_t *lists = reinterpret_cast<int32_t *>(st + pbytes);
  // the lists back to back (an empty list's data() may be null: no copy)
  for (const std::vector<int32_t> *l : {&rt.pf, &rt.row, &rt.chunk, &rt.large, &rt.mid, &rt.lfast}) {
    if (!l->empty()) memcpy(lists, l->data(), sizeof(int32_t) * l->size());
    lists += l->size();
  }
  HS_HIP(hipMemcpyAsync(ctx->plans.p, st, bytes, hipMemcpyHostToDevice, stream));
  HS_HIP(hipEventRecord(ctx->plan_done, stream));
  ctx->plan_pending = true;
  try {
    ctx->last_plans = plans;
  } catch (const std::bad_alloc &) {
    ctx->last_plans.clear();
    return fail(HS_ERR_OUT_OF_MEMORY, "host allocation failed");
  }
  ctx->last_vocab = vocab;
  return HS_OK;
}

// Workgroups per row for `rows` rows streamed one workgroup per part: small
// batches split each row (parts of whole float4s) so that the launch fills the
// CUs.  HS_ROW_SPLIT (read at context creation) forces the count, whatever
// the part size.  Every part holds at least one float4.
int choose_split(const hs_context *ctx, int rows, int vocab) {
  if (rows <= 0) return 1;
  int split = ctx->row_split > 0 ? ctx->row_split
                                 : std::min(hs::kSplitCUs / rows, vocab / hs::kSplitMinPart);
  const int nf4 = (vocab + 3) / 4;
  split = std::max(1, std::min(split, std::min(hs::kSplitMax, nf4)));
  while (split > 1 && (split - 1) * ((nf4 + split - 1) / split) >= nf4) --split;
  return split;
}

// The split rows' hand-over buffers for rows x split parts.
// A buffer that holds zeros between calls (arrival counters), grown and
// cleared together: a failed clear drops the buffer, so that the next call
// allocates and clears it again instead of counting from stale values.
// Grows a counter buffer and clears it on the call's stream, ahead of the
// call's kernels (a blocking-stream hipMemset would not be ordered with the
// context's non-blocking stream, and the first kernels could count into
// memory not yet cleared).  The clear is a fill kernel, not a memset node.
int ensure_zeroed(DevBuf &b, size_t need, hipStream_t stream) {
  if (b.bytes >= need) return HS_OK;
  HS_HIP(b.ensure(need));
  const hipError_t e = inject_failure()
                           ? hipErrorOutOfMemory
                           : hs::launch_fill_u32(static_cast<uint32_t *>(b.p),
                                                 (int64_t)(b.bytes / sizeof(uint32_t)), 0u, stream);
  if (e != hipSuccess) {
    b.release();
    return fail(HS_ERR_HIP, "hipMemset(counters) failed: %s", hipGetErrorString(e));
  }
  return HS_OK;
}

int ensure_split(hs_context *ctx, int rows, int split, hipStream_t stream) {
  if (split <= 1) return HS_OK;
  const size_t parts = (size_t)rows * (size_t)split;
  HS_HIP(ctx->split_list.ensure(parts * hs::kPartCap * sizeof(unsigned long long)));
  HS_HIP(ctx->split_meta.ensure(parts * sizeof(hs::SplitMeta)));
  return ensure_zeroed(ctx->split_cnt, sizeof(uint32_t) * (size_t)rows, stream);
}

hs::Workspace split_workspace(const hs_context *ctx) {
  hs::Workspace ws;
  memset(&ws, 0, sizeof ws);
  ws.split_list = static_cast<unsigned long long *>(ctx->split_list.p);
  ws.split_meta = static_cast<hs::SplitMeta *>(ctx->split_meta.p);
  ws.split_cnt = static_cast<uint32_t *>(ctx->split_cnt.p);
  return ws;
}

// With timing on, takes start/end events for every kernel the call launches.
int begin_timed(hs_context *ctx, const hs::LaunchArgs &a, hipEvent_t **ev) {
  *ev = nullptr;
  if (!ctx->timing) return HS_OK;
  hs_context::TimedCall tc{};
  tc.mask = hs::launched_kernels(a);
  for (int i = 0; i < 2 * hs::kTimedKernels; ++i) {
    if (!(tc.mask >> (i / 2) & 1u)) continue;
    if (ctx->ev_free.empty()) {
      hipEvent_t x;
      HS_HIP(hipEventCreate(&x));
      ctx->ev_free.push_back(x);
    }
    tc.ev[i] = ctx->ev_free.back();
    ctx->ev_free.pop_back();
  }
  ctx->timed.push_back(tc);
  *ev = ctx->timed.back().ev;
  return HS_OK;
}

// A failed launch may have left counters of earlier kernels of the call
// raised: clear them for the next call.
void reset_counters(hs_context *ctx, hipStream_t stream) {
  for (DevBuf *b : {&ctx->cand_count, &ctx->split_cnt})
    if (b->p)
      (void)hs::launch_fill_u32(static_cast<uint32_t *>(b->p),
                                (int64_t)(b->bytes / sizeof(uint32_t)), 0u, stream);
}

int sample_device(hs_context *ctx, float *d_logits, int32_t rows, int64_t row_stride,
                  int32_t vocab, const int32_t *d_hist_ids, const int64_t *d_hist_offsets,
                  const hs_sample_config *configs, const double *d_uniforms, int32_t *d_tokens,
                  int32_t cand_stride, int32_t *d_cand_ids, float *d_cand_probs,
                  int32_t *d_cand_count, int32_t *d_cutoff, uint32_t *d_row_flags,
                  hipStream_t stream, const int64_t *d_hist_len = nullptr, int64_t hist_cap = 0,
                  const hs::DecodeArgs *dec = nullptr) {
  if (!ctx) return fail(HS_ERR_INVALID_ARGUMENT, "null context");
  if (rows < 0) return fail(HS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %d)", rows);
  if (rows == 0) return HS_OK;
  if (!configs || !d_uniforms || !d_tokens)
    return fail(HS_ERR_INVALID_ARGUMENT, "configs, uniforms and tokens must not be null");
  if (hist_cap == 0 && (d_hist_ids == nullptr) != (d_hist_offsets == nullptr))
    return fail(HS_ERR_INVALID_ARGUMENT, "history ids and offsets must both be given or both null");
  if (cand_stride < 0) return fail(HS_ERR_INVALID_ARGUMENT, "cand_stride must be >= 0");
  if ((d_cand_ids || d_cand_probs) && cand_stride == 0)
    return fail(HS_ERR_INVALID_ARGUMENT, "candidate outputs need cand_stride > 0");
  DeviceGuard guard(ctx->device);
  int rc0 = enter_stream(ctx, stream);
  if (rc0) return rc0;
  if (vocab <= 0) {
    // src/sampler.ts: no logit is read; every path returns 0.
    HS_HIP(hipMemsetAsync(d_tokens, 0, sizeof(int32_t) * (size_t)rows, stream));
    if (d_cand_count) HS_HIP(hipMemsetAsync(d_cand_count, 0, sizeof(int32_t) * rows, stream));
    if (d_cutoff) HS_HIP(hipMemsetAsync(d_cutoff, 0, sizeof(int32_t) * rows, stream));
    if (d_row_flags) HS_HIP(hipMemsetAsync(d_row_flags, 0, sizeof(uint32_t) * rows, stream));
    if (dec) {   // the drawn 0s go through the decode bookkeeping
      const hipError_t e = hs::launch_decode_append(*dec, stream);
      if (e != hipSuccess)
        return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
    }
    return leave_stream(ctx, stream, false);
  }
  if (!d_logits) return fail(HS_ERR_INVALID_ARGUMENT, "logits must not be null");
  if (row_stride < vocab)
    return fail(HS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  const int64_t S = (vocab + hs::kChunk - 1) / hs::kChunk;
  if (S * hs::kChunkCap > 0x7FFFFFFF / 2 || (int64_t)rows * S > 0x7FFFFFFF)
    return fail(HS_ERR_UNSUPPORTED, "vocab %d x rows %d too large", vocab, rows);

  std::vector<hs::RowPlan> &plans = ctx->call_plans;
  Routing &rt = ctx->call_rt;
  try {
    int rc = build_plans(configs, rows, vocab, ctx->row_min_rows, plans, rt);
    if (rc) return rc;
  } catch (const std::bad_alloc &) {
    return fail(HS_ERR_OUT_OF_MEMORY, "host allocation failed");
  }
  const int n_pf = (int)rt.pf.size(), n_row = (int)rt.row.size(), n_chunk = (int)rt.chunk.size();
  const int n_large = (int)rt.large.size(), n_mid = (int)rt.mid.size();
  const int n_lfast = (int)rt.lfast.size();

  // workspace (the chunk path only)
  if (n_chunk > 0) {
    HS_HIP(ctx->cand.ensure((size_t)n_chunk * (size_t)S * hs::kChunkCap * sizeof(uint2)));
    HS_HIP(ctx->info.ensure((size_t)n_chunk * (size_t)S * sizeof(hs::ChunkInfo)));
    const int rz = ensure_zeroed(ctx->cand_count, sizeof(int32_t) * (size_t)n_chunk, stream);
    if (rz) return rz;
  }
  if (n_lfast > 0) HS_HIP(ctx->large_retry.ensure(sizeof(int32_t) * (size_t)n_lfast));
  if (n_large > 0) HS_HIP(ctx->large_replay.ensure(sizeof(hs::ReplayReq) * (size_t)n_large));
  // a large-k row whose slots exceed the LDS replay's, or candidate outputs
  // longer than it orders, may need the device-memory replay: one region of
  // vocab keys and vocab ids per workgroup of it
  int replay_dev = 0;
  {
    bool big = (d_cand_ids || d_cand_probs) && cand_stride > hs::kReplayCands;
    for (int32_t r : rt.large) big |= plans[(size_t)r].k > hs::kReplayMaxK;
    if (big && n_large > 0) {
      replay_dev = std::min(n_large, hs::kReplayDevBlocks);
      HS_HIP(ctx->replay_slots.ensure((size_t)replay_dev * ((size_t)vocab * 8 +
                                                           (size_t)(vocab + 63) / 64 * 8)));
    }
  }
  // small batches split each row of the row kernel over several workgroups
  const int split = choose_split(ctx, n_row, vocab);
  int rc = ensure_split(ctx, n_row, split, stream);
  if (rc) return rc;
  rc = upload_plans(ctx, plans, rt, vocab, stream);
  if (rc) return rc;

  hs::Workspace ws = split_workspace(ctx);
  ws.plans = static_cast<hs::RowPlan *>(ctx->plans.p);
  const int32_t *lists = reinterpret_cast<const int32_t *>(ws.plans + rows);
  ws.pf_list = lists;
  ws.row_list = lists + n_pf;
  ws.chunk_list = lists + n_pf + n_row;
  ws.large_list = lists + n_pf + n_row + n_chunk;
  ws.mid_list = lists + n_pf + n_row + n_chunk + n_large;
  ws.lfast_list = lists + n_pf + n_row + n_chunk + n_large + n_mid;
  ws.large_retry = static_cast<int32_t *>(ctx->large_retry.p);
  ws.large_replay = static_cast<hs::ReplayReq *>(ctx->large_replay.p);
  if (replay_dev > 0) {
    ws.replay_keys = static_cast<uint32_t *>(ctx->replay_slots.p);
    ws.replay_ids = reinterpret_cast<int32_t *>(ws.replay_keys + (size_t)replay_dev * vocab);
    ws.replay_lvl1 = reinterpret_cast<unsigned long long *>(ws.replay_ids + (size_t)replay_dev * vocab);
  }
  ws.cand = static_cast<uint2 *>(ctx->cand.p);
  ws.cand_count = static_cast<int32_t *>(ctx->cand_count.p);
  ws.info = static_cast<hs::ChunkInfo *>(ctx->info.p);

  hs::LaunchArgs a;
  memset(&a, 0, sizeof a);
  a.logits = d_logits;
  a.stride = row_stride;
  a.rows = rows;
  a.vocab = vocab;
  a.chunks = (int32_t)S;
  a.vec = ((reinterpret_cast<uintptr_t>(d_logits) & 15u) == 0 && (row_stride & 3) == 0) ? 1 : 0;
  a.want_cands = (d_cand_ids || d_cand_probs) ? 1 : 0;
  a.n_pf = n_pf;
  a.n_row = n_row;
  a.split = split;
  a.rows_direct = n_row == rows ? 1 : 0;
  a.n_chunk = n_chunk;
  a.n_large = n_large;
  a.n_mid = n_mid;
  a.n_lfast = n_lfast;
  a.replay_dev = replay_dev;
  a.hist_ids = d_hist_ids;
  a.hist_off = d_hist_offsets;
  a.hist_len = d_hist_len;
  a.hist_cap = hist_cap;
  if (dec) {
    a.dec_ring = dec->ring;
    a.dec_len = dec->len;
    a.dec_done = dec->done;
    a.dec_stop = dec->stop_ids;
    a.dec_nstop = dec->n_stop;
  }
  a.uniforms = d_uniforms;
  a.tokens = d_tokens;
  a.cand_stride = cand_stride;
  a.cand_ids = d_cand_ids;
  a.cand_probs = d_cand_probs;
  a.cand_count_out = d_cand_count;
  a.cutoff_out = d_cutoff;
  a.row_flags = d_row_flags;
  hipEvent_t *ev = nullptr;
  rc = begin_timed(ctx, a, &ev);
  if (rc) return rc;
  hipError_t e = hs::launch_sample(a, ws, stream, ev, ctx->done_ev);
  if (e != hipSuccess) {
    reset_counters(ctx, stream);
    (void)leave_stream(ctx, stream, false);
    return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  }
  return leave_stream(ctx, stream, ev == nullptr);
}

// src/kernels.ts:1613-1654 (the argmax pipeline of the engine's greedy route).
int argmax_device(hs_context *ctx, const float *d_logits, int32_t rows, int64_t row_stride,
                  int32_t vocab, int32_t *d_tokens, hipStream_t stream) {
  if (!ctx) return fail(HS_ERR_INVALID_ARGUMENT, "null context");
  if (rows < 0) return fail(HS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %d)", rows);
  if (rows == 0) return HS_OK;
  if (!d_tokens) return fail(HS_ERR_INVALID_ARGUMENT, "tokens must not be null");
  DeviceGuard guard(ctx->device);
  int rc0 = enter_stream(ctx, stream);
  if (rc0) return rc0;
  if (vocab <= 0) {   // no invocation scans an id: every slot keeps id 0
    HS_HIP(hipMemsetAsync(d_tokens, 0, sizeof(int32_t) * (size_t)rows, stream));
    return leave_stream(ctx, stream, false);
  }
  if (!d_logits) return fail(HS_ERR_INVALID_ARGUMENT, "logits must not be null");
  if (row_stride < vocab)
    return fail(HS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  if (vocab > hs::kArgmaxMaxVocab)
    return fail(HS_ERR_UNSUPPORTED, "vocab %d above %d", vocab, hs::kArgmaxMaxVocab);
  const int split = choose_split(ctx, rows, vocab);
  if ((int64_t)rows * split > 0x7FFFFFFF)
    return fail(HS_ERR_UNSUPPORTED, "rows %d too many", rows);
  int rc = ensure_split(ctx, rows, split, stream);
  if (rc) return rc;
  hs::Workspace ws = split_workspace(ctx);
  hs::LaunchArgs a;
  memset(&a, 0, sizeof a);
  a.logits = const_cast<float *>(d_logits);   // read only
  a.stride = row_stride;
  a.rows = rows;
  a.vocab = vocab;
  a.vec = ((reinterpret_cast<uintptr_t>(d_logits) & 15u) == 0 && (row_stride & 3) == 0) ? 1 : 0;
  a.n_argmax = rows;
  a.split = split;
  a.rows_direct = 1;
  a.tokens = d_tokens;
  hipEvent_t *ev = nullptr;
  rc = begin_timed(ctx, a, &ev);
  if (rc) return rc;
  hipError_t e = hs::launch_sample(a, ws, stream, ev, ctx->done_ev);
  if (e != hipSuccess) {
    reset_counters(ctx, stream);
    (void)leave_stream(ctx, stream, false);
    return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  }
  return leave_stream(ctx, stream, ev == nullptr);
}

// src/engine.ts:1493-1515 (the lm_head GEMV; see lmhead_kernels.hip).
// The checks and arguments of an lm_head GEMV call, on the call's stream
// (entered: enter_stream ran).  A Hadamard-folded weight's input is rotated
// here, into the workspace.  *skip: nothing to compute (M or N is 0).
int gemv_setup(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx, const hs_weights *wt,
               float *d_y, int64_t ldy, hipStream_t stream, hs::GemvArgs &g, bool *skip) {
  *skip = false;
  if (!ctx) return fail(HS_ERR_INVALID_ARGUMENT, "null context");
  if (!wt) return fail(HS_ERR_INVALID_ARGUMENT, "null weights");
  const int32_t K = wt->cols, N = wt->rows, w_type = wt->type;
  const void *d_w = wt->data;
  if (M < 0 || N < 0 || K <= 0)
    return fail(HS_ERR_INVALID_ARGUMENT, "need M >= 0, N >= 0, K > 0 (got %d, %d, %d)", M, N, K);
  if (M == 0 || N == 0) {
    *skip = true;
    return HS_OK;
  }
  if (!d_x || !d_w || !d_y) return fail(HS_ERR_INVALID_ARGUMENT, "x, w and y must not be null");
  if (ldx < K || ldy < N)
    return fail(HS_ERR_INVALID_ARGUMENT, "ldx %lld < K or ldy %lld < N", (long long)ldx, (long long)ldy);
  int bw = 0, bb = 0;
  const bool planar = hs::tern_quant_bytes(w_type) > 0;
  switch (w_type) {
    case hs::kW_F32: bw = 32; bb = 128; break;   // as 32-weight units
    case hs::kW_Q4_0: bw = 32; bb = 18; break;
    case hs::kW_Q4_1: bw = 32; bb = 20; break;
    case hs::kW_Q4_K: bw = 256; bb = 144; break;
    case hs::kW_Q6_K: bw = 256; bb = 210; break;
    case hs::kW_Q1_0: case hs::kW_PQ2_0: case hs::kW_PTQ1_0:
      bw = 128; bb = hs::tern_quant_bytes(w_type); break;
    default: return fail(HS_ERR_UNSUPPORTED, "weight type %d is not supported", w_type);
  }
  if (K % bw)
    return fail(HS_ERR_INVALID_ARGUMENT, "K %d is not a multiple of the block size %d", K, bw);
  if (K > hs::kGemvMaxK) return fail(HS_ERR_UNSUPPORTED, "K %d above %d", K, hs::kGemvMaxK);
  if (planar && !wt->scales16)
    return fail(HS_ERR_INVALID_ARGUMENT, "weight type %d needs its binary16 scales", w_type);
  if (!planar && wt->scales16)
    return fail(HS_ERR_INVALID_ARGUMENT, "scales16 is for types 41, 142 and 143 only");
  if (wt->hadamard && K % 512)
    return fail(HS_ERR_INVALID_ARGUMENT, "a Hadamard-folded weight needs K %% 512 == 0 (K = %d)", K);
  const uintptr_t walign = planar ? (w_type == hs::kW_PTQ1_0 ? 3u : 15u) : 15u;
  if ((reinterpret_cast<uintptr_t>(d_w) & walign) || (reinterpret_cast<uintptr_t>(d_x) & 3u) ||
      (reinterpret_cast<uintptr_t>(wt->scales16) & 3u))
    return fail(HS_ERR_INVALID_ARGUMENT,
                "w must be 16-byte (PTQ1_0 quants 4-byte), scales and x 4-byte aligned");
  const int64_t row_bytes = (int64_t)(K / bw) * bb;
  // (Q6_K's slabs read up to 3 KiB past a row's start)
  if ((int64_t)N * row_bytes > (w_type == hs::kW_Q6_K ? 0xFFFF0000LL : 0xFFFFFF00LL))
    return fail(HS_ERR_UNSUPPORTED, "weights of %lld bytes above 4 GiB", (long long)(N * row_bytes));
  memset(&g, 0, sizeof g);
  g.x = d_x;
  g.ldx = ldx;
  g.w = d_w;
  g.scales = wt->scales16;
  g.s_bytes = planar ? (uint32_t)((int64_t)N * (K / 128) * 2) : 0u;
  g.w_bytes = (uint32_t)(N * row_bytes);
  g.row_bytes = (uint32_t)row_bytes;
  g.y = d_y;
  g.ldy = ldy;
  g.N = N;
  g.K = K;
  g.M = M;
  g.type = w_type;
  g.units = w_type == hs::kW_Q6_K ? K / 64 : K / 32;
  g.nru = g.units <= 64 ? 1 : 2;
  int seg = 1;
  while (seg < g.units && seg < 64) seg <<= 1;
  g.seg = g.nru == 1 ? seg : 64;
  const int64_t steps = ((int64_t)N + 64 / g.seg - 1) / (64 / g.seg);
  // at most one wave per row step (the launch caps it at the resident workgroups)
  const int64_t wpb = hs::kGemvThreads / 64;
  g.blocks = (int32_t)std::min<int64_t>((steps + wpb - 1) / wpb, 1 << 20);
  if (M > 65535) return fail(HS_ERR_UNSUPPORTED, "M %d above 65535", M);
  if (w_type == hs::kW_Q6_K || w_type == hs::kW_Q4_K) {   // the hand-over slots of tiles cut between waves
    int cus = 0;
    HS_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device));
    g.part_cap = cus * hs::kGemvWavesPerCU;
    const size_t slots = (size_t)g.part_cap * (size_t)M;
    HS_HIP(ctx->gemv_part.ensure(slots * 16 * sizeof(float)));
    const int rz = ensure_zeroed(ctx->gemv_cnt, slots * sizeof(uint32_t), stream);
    if (rz) return rz;
    g.part = static_cast<float *>(ctx->gemv_part.p);
    g.tile_cnt = static_cast<uint32_t *>(ctx->gemv_cnt.p);
  }
  if (wt->hadamard) {   // src/engine.ts:1121-1145: the input is rotated first
    HS_HIP(ctx->gemv_rot.ensure((size_t)M * (size_t)K * sizeof(float)));
    float *rot = static_cast<float *>(ctx->gemv_rot.p);
    const hipError_t e = hs::launch_hadamard(d_x, ldx, wt->signs, rot, M, K, stream);
    if (e != hipSuccess) return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
    g.x = rot;
    g.ldx = K;
  }
  return HS_OK;
}

// Start/end events of timing slot `slot` for the call's one kernel, when
// timing is on (null otherwise).
int timed_slot(hs_context *ctx, int slot, hipEvent_t **ev) {
  *ev = nullptr;
  if (!ctx->timing) return HS_OK;
  hs_context::TimedCall tc{};
  tc.mask = 1u << slot;
  for (int i = 0; i < 2; ++i) {
    if (ctx->ev_free.empty()) {
      hipEvent_t x;
      HS_HIP(hipEventCreate(&x));
      ctx->ev_free.push_back(x);
    }
    tc.ev[2 * slot + i] = ctx->ev_free.back();
    ctx->ev_free.pop_back();
  }
  ctx->timed.push_back(tc);
  *ev = ctx->timed.back().ev + 2 * slot;
  return HS_OK;
}

int gemv_device(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx, const hs_weights *wt,
                float *d_y, int64_t ldy, hipStream_t stream) {
  if (!ctx) return fail(HS_ERR_INVALID_ARGUMENT, "null context");
  DeviceGuard guard(ctx->device);
  int rc = enter_stream(ctx, stream);
  if (rc) return rc;
  hs::GemvArgs g;
  bool skip = false;
  rc = gemv_setup(ctx, d_x, M, ldx, wt, d_y, ldy, stream, g, &skip);
  if (rc || skip) return rc;   // nothing was enqueued
  hipEvent_t *ev = nullptr;
  rc = timed_slot(ctx, hs::kGemvTimedSlot, &ev);
  if (rc) return rc;
  const hipError_t e = hs::launch_gemv(g, stream, ev, ctx->done_ev);
  if (e != hipSuccess) {
    (void)leave_stream(ctx, stream, false);
    return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  }
  return leave_stream(ctx, stream, ev == nullptr);
}

// Plans and routing lists written into fixed arrays (no allocation): the
// lists pf | row | large | mid | two-pass large back to back, in row order,
// their lengths in n[0..4], and in n[5] whether a row of the large list has
// more slots than the LDS replay holds.  Routing as build_plans with every
// row on the one-pass kernels (vocab <= kRowMaxVocab): rows with k <= 64
// join the mid kernel's launch when it has rows.
void build_plans_fixed(const hs_sample_config *cfgs, int rows, int vocab, hs::RowPlan *plans,
                       int32_t *lists, int n[6]) {
  int n_pf = 0, n_row = 0, n_large = 0, n_mid = 0, n_small = 0, n_lfast = 0, big = 0;
  for (int r = 0; r < rows; ++r) {
    const hs::RowPlan p = plan_row(cfgs[r], vocab);
    plans[r] = p;
    n_lfast += two_pass_large(p, vocab);
    n_large += p.mode == hs::kModeLarge && !two_pass_large(p, vocab);
    big |= p.mode == hs::kModeLarge && !two_pass_large(p, vocab) && p.k > hs::kReplayMaxK;
    n_mid += p.mode == hs::kModeGeneric;
    n_row += p.mode == hs::kModeGreedy || p.mode == hs::kModeSmall;
    n_small += p.mode == hs::kModeSmall;
  }
  const bool merge = n_mid > 0 && n_row > 0;
  if (merge) {
    n_row -= n_small;
    n_mid += n_small;
  }
  auto to_mid = [&](const hs::RowPlan &p) {
    return p.mode == hs::kModeGeneric || (merge && p.mode == hs::kModeSmall);
  };
  for (int r = 0; r < rows; ++r) n_pf += in_prepass(plans[r], to_mid(plans[r]));
  int32_t *pf = lists, *row = pf + n_pf, *large = row + n_row, *mid = large + n_large;
  int32_t *lfast = mid + n_mid;
  for (int r = 0; r < rows; ++r) {
    const hs::RowPlan &p = plans[r];
    if (in_prepass(p, to_mid(p))) *pf++ = r;
    if (two_pass_large(p, vocab)) *lfast++ = r;
    else if (p.mode == hs::kModeLarge) *large++ = r;
    else if (to_mid(p)) *mid++ = r;
    else *row++ = r;
  }
  n[0] = n_pf;
  n[1] = n_row;
  n[2] = n_large;
  n[3] = n_mid;
  n[4] = n_lfast;
  n[5] = big;
}

// hs_sample_batch_device with the device's `scratch` array as its workspace:
// no allocation of any kind.  The plans go through the context's pinned
// staging (set up at creation) and are not uploaded again while this
// context's last upload is the latest one into the device's scratch and the
// configs, rows and vocab are unchanged.
int sample_device_noalloc(hs_context *ctx, float *d_logits, int32_t rows, int64_t row_stride,
                          int32_t vocab, const int32_t *d_hist_ids, const int64_t *d_hist_offsets,
                          const hs_sample_config *configs, const double *d_uniforms,
                          int32_t *d_tokens, hipStream_t stream) {
  if (rows < 0) return fail(HS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %d)", rows);
  if (rows == 0) return HS_OK;
  if (!configs || !d_uniforms || !d_tokens)
    return fail(HS_ERR_INVALID_ARGUMENT, "configs, uniforms and tokens must not be null");
  if ((d_hist_ids == nullptr) != (d_hist_offsets == nullptr))
    return fail(HS_ERR_INVALID_ARGUMENT, "history ids and offsets must both be given or both null");
  if (rows > na::kMaxRows)
    return fail(HS_ERR_UNSUPPORTED, "rows %d above the no-allocation limit %d", rows, na::kMaxRows);
  if (vocab > hs::kRowMaxVocab)
    return fail(HS_ERR_UNSUPPORTED, "vocab %d above the no-allocation limit %d", vocab,
                hs::kRowMaxVocab);
  if (ctx->device < 0 || ctx->device >= na::kMaxDevices || !g_scratch[ctx->device] ||
      !ctx->na_staging || !ctx->na_last)
    return fail(HS_ERR_UNSUPPORTED, "no scratch workspace on device %d", ctx->device);
  DeviceGuard guard(ctx->device);
  // The call blocks on its last upload's event when the configs change and
  // reads plans from the shared scratch that later calls rewrite: it cannot
  // be captured into a graph.  Checked before anything is enqueued.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HS_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(HS_ERR_UNSUPPORTED, "the no-allocation entry point cannot be captured into a graph");
  int rc = enter_stream(ctx, stream);
  if (rc) return rc;
  if (vocab <= 0) {   // src/sampler.ts: no logit is read; every path returns 0
    const hipError_t e = hs::launch_fill_u32(reinterpret_cast<uint32_t *>(d_tokens), rows, 0u, stream);
    if (e != hipSuccess) return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
    return leave_stream(ctx, stream, false);
  }
  if (!d_logits) return fail(HS_ERR_INVALID_ARGUMENT, "logits must not be null");
  if (row_stride < vocab)
    return fail(HS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  char *base = static_cast<char *>(g_scratch[ctx->device]);
  std::atomic<uint64_t> &gen = g_scratch_gen[ctx->device];
  const size_t cbytes = sizeof(hs_sample_config) * (size_t)rows;
  const bool same = ctx->na_gen == gen.load() && ctx->na_rows == rows && ctx->na_vocab == vocab &&
                    memcmp(ctx->na_last, configs, cbytes) == 0;
  if (!same) {
    if (ctx->na_pending) {   // the staging may still be read by the last upload
      HS_HIP(hipEventSynchronize(ctx->na_upload_ev));
      ctx->na_pending = false;
    }
    // Invalidate first: once the scratch may hold new plans, no context
    // (this one included) may take the `same` path on its old bookkeeping,
    // even if a copy below fails.
    ++gen;
    ctx->na_gen = ~0ull;
    ctx->na_rows = -1;
    char *st = static_cast<char *>(ctx->na_staging);
    hs::RowPlan *plans = reinterpret_cast<hs::RowPlan *>(st);
    int32_t *lists = reinterpret_cast<int32_t *>(st + na::kPlansBytes);
    build_plans_fixed(configs, rows, vocab, plans, lists, ctx->na_count);
    const int nl = ctx->na_count[0] + ctx->na_count[1] + ctx->na_count[2] + ctx->na_count[3] +
                   ctx->na_count[4];
    // a failure after the first copy was issued waits for the stream, so
    // that no copy still reads the staging when the next call refills it
    hipError_t ue = inject_failure() ? hipErrorOutOfMemory
                                     : hipMemcpyAsync(base + na::kPlansOff, plans,
                                                      sizeof(hs::RowPlan) * (size_t)rows,
                                                      hipMemcpyHostToDevice, stream);
    if (ue != hipSuccess)
      return fail(HS_ERR_HIP, "hipMemcpyAsync(plans) failed: %s", hipGetErrorString(ue));
    ue = inject_failure() ? hipErrorOutOfMemory
                          : hipMemcpyAsync(base + na::kListsOff, lists, sizeof(int32_t) * (size_t)nl,
                                           hipMemcpyHostToDevice, stream);
    if (ue == hipSuccess)
      ue = inject_failure() ? hipErrorOutOfMemory : hipEventRecord(ctx->na_upload_ev, stream);
    if (ue != hipSuccess) {
      (void)hipStreamSynchronize(stream);
      return fail(HS_ERR_HIP, "plan upload failed: %s", hipGetErrorString(ue));
    }
    ctx->na_pending = true;
    memcpy(ctx->na_last, configs, cbytes);
    ctx->na_rows = rows;
    ctx->na_vocab = vocab;
    ctx->na_gen = ++gen;
  }
  const int n_pf = ctx->na_count[0], n_row = ctx->na_count[1], n_large = ctx->na_count[2],
            n_mid = ctx->na_count[3], n_lfast = ctx->na_count[4];
  const int replay_dev = n_large > 0 && ctx->na_count[5] ? 1 : 0;
  // small batches split each row of the row kernel (at most kSplitCUs parts)
  int split = choose_split(ctx, n_row, vocab);
  while (split > 1 && (int64_t)n_row * split > hs::kSplitCUs) --split;

  hs::Workspace ws;
  memset(&ws, 0, sizeof ws);
  ws.plans = reinterpret_cast<hs::RowPlan *>(base + na::kPlansOff);
  const int32_t *lists = reinterpret_cast<const int32_t *>(base + na::kListsOff);
  ws.pf_list = lists;
  ws.row_list = lists + n_pf;
  ws.chunk_list = lists + n_pf + n_row;
  ws.large_list = lists + n_pf + n_row;
  ws.mid_list = lists + n_pf + n_row + n_large;
  ws.lfast_list = lists + n_pf + n_row + n_large + n_mid;
  ws.large_retry = reinterpret_cast<int32_t *>(base + na::kRetryOff);
  ws.large_replay = reinterpret_cast<hs::ReplayReq *>(base + na::kReplayOff);
  ws.split_list = reinterpret_cast<unsigned long long *>(base + na::kSplitListOff);
  ws.split_meta = reinterpret_cast<hs::SplitMeta *>(base + na::kSplitMetaOff);
  ws.split_cnt = reinterpret_cast<uint32_t *>(base + na::kSplitCntOff);
  ws.replay_keys = reinterpret_cast<uint32_t *>(base + na::kRKeysOff);
  ws.replay_ids = reinterpret_cast<int32_t *>(base + na::kRIdsOff);
  ws.replay_lvl1 = reinterpret_cast<unsigned long long *>(base + na::kRLvl1Off);

  hs::LaunchArgs a;
  memset(&a, 0, sizeof a);
  a.logits = d_logits;
  a.stride = row_stride;
  a.rows = rows;
  a.vocab = vocab;
  a.chunks = (int32_t)((vocab + hs::kChunk - 1) / hs::kChunk);
  a.vec = ((reinterpret_cast<uintptr_t>(d_logits) & 15u) == 0 && (row_stride & 3) == 0) ? 1 : 0;
  a.n_pf = n_pf;
  a.n_row = n_row;
  a.split = split;
  a.rows_direct = n_row == rows ? 1 : 0;
  a.n_large = n_large;
  a.n_mid = n_mid;
  a.n_lfast = n_lfast;
  a.replay_dev = replay_dev;
  a.hist_ids = d_hist_ids;
  a.hist_off = d_hist_offsets;
  a.uniforms = d_uniforms;
  a.tokens = d_tokens;
  const hipError_t e = hs::launch_sample(a, ws, stream, nullptr, ctx->done_ev);
  if (e != hipSuccess) {
    // a kernel that did not run may leave a split counter raised
    (void)hs::launch_fill_u32(ws.split_cnt, hs::kSplitCUs, 0u, stream);
    (void)leave_stream(ctx, stream, false);
    return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  }
  return leave_stream(ctx, stream, true);
}

// hs_sample_logits_batch for small blocks whose rows all stream their logits
// once: the kernels read the logits, uniforms and histories from the
// context's pinned buffer and write the tokens and the penalised logits
// there (device access to pinned host memory), so the call makes no copy to
// or from device memory.  ctx->gidx lists the penalised entries.
int sample_host_zero_copy(hs_context *ctx, float *logits, size_t lbytes, int32_t rows,
                          int64_t row_stride, int32_t vocab, const int32_t *hist_ids,
                          const int64_t *hist_offsets, int64_t hist_total,
                          const hs_sample_config *configs, const double *uniforms,
                          int32_t *tokens_out) {
  hipStream_t st = ctx->stream;
  const size_t s_u = sizeof(double) * rows;
  const size_t s_off = hist_offsets ? sizeof(int64_t) * (size_t)(rows + 1) : 0;
  const size_t s_hist = sizeof(int32_t) * (size_t)hist_total;
  const size_t o_u = pin_align(lbytes);
  const size_t o_off = o_u + pin_align(s_u);
  const size_t o_hist = o_off + pin_align(s_off);
  const size_t o_tok = o_hist + pin_align(s_hist);
  HS_HIP(ctx->h_pin.ensure(o_tok + sizeof(int32_t) * rows));
  char *pin = static_cast<char *>(ctx->h_pin.p);
  memcpy(pin, logits, lbytes);
  memcpy(pin + o_u, uniforms, s_u);
  if (hist_offsets) {
    memcpy(pin + o_off, hist_offsets, s_off);
    if (hist_total > 0) memcpy(pin + o_hist, hist_ids, s_hist);
  }
  float *p_logits = reinterpret_cast<float *>(pin);
  const int rc = sample_device(
      ctx, p_logits, rows, row_stride, vocab,
      hist_offsets ? reinterpret_cast<const int32_t *>(pin + o_hist) : nullptr,
      hist_offsets ? reinterpret_cast<const int64_t *>(pin + o_off) : nullptr, configs,
      reinterpret_cast<const double *>(pin + o_u), reinterpret_cast<int32_t *>(pin + o_tok), 0,
      nullptr, nullptr, nullptr, nullptr, nullptr, st);
  // the pinned buffer is free again only once the stream has drained: after
  // a call that launched, once done_ev (its last kernel's completion) has
  // completed, which hipEventSynchronize returns about 4 us sooner than
  // hipStreamSynchronize on a stream whose last kernel carries that event
  const bool last_event = rc == HS_OK && ctx->has_done && ctx->done_stream == st;
  const hipError_t es = last_event ? hipEventSynchronize(ctx->done_ev) : hipStreamSynchronize(st);
  if (rc) return rc;
  if (es != hipSuccess)
    return fail(HS_ERR_HIP, "synchronisation failed: %s", hipGetErrorString(es));
  memcpy(tokens_out, pin + o_tok, sizeof(int32_t) * rows);
  for (const int64_t g : ctx->gidx) logits[g] = p_logits[g];
  for (int r = 0; r < rows; ++r)
    if (tokens_out[r] < 0)
      return fail(HS_ERR_UNSUPPORTED,
                  "row %d: top-k above %d with equal logits at the drawn position; the "
                  "reference orders them by its slot history, which this build replays up to "
                  "that top-k only", r, hs::kReplayDevMaxK);
  return HS_OK;
}

}  // namespace

// Every entry point that uses a context holds its mutex for the whole call.
#define HS_LOCK(ctx)                                                   \
  if (!(ctx)) return fail(HS_ERR_INVALID_ARGUMENT, "null context");    \
  std::lock_guard<std::mutex> hs_lock_((ctx)->mu)

extern "C" {

int hs_abi_version(void) { return HS_ABI_VERSION; }

const char *hs_last_error(void) { return g_error.c_str(); }

void hs_config_default(hs_sample_config *c) {
  if (!c) return;
  c->temperature = 0.6;
  c->top_k = 20.0;
  c->top_p = 0.95;
  c->min_p = 0.0;
  c->repetition_penalty = 1.0;
  c->presence_penalty = 0.0;
  c->frequency_penalty = 0.0;
}

int hs_context_create(int device, hs_context **out) {
  if (!out) return fail(HS_ERR_INVALID_ARGUMENT, "out must not be null");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return fail(HS_ERR_HIP, "no HIP device available (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n)
    return fail(HS_ERR_INVALID_ARGUMENT, "device %d out of range [0, %d)", device, n);
  if (const char *env = getenv("HS_INJECT_HIP_FAILURE")) g_inject.store(atoi(env));
  DeviceGuard guard(device);
  {
    std::lock_guard<std::mutex> lk(g_prep_mu);
    bool done = false;
    for (int d : g_prepared) done |= d == device;
    if (!done) {
      HS_HIP(hs::prepare_kernels());
      if (device < na::kMaxDevices) {
        // the no-allocation entry point's workspace on this device: its
        // address here, once; its arrival counters start at zero
        void *p = nullptr;
        HS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        HS_HIP(hipMemset(static_cast<char *>(p) + na::kSplitCntOff, 0, na::kSplitCntBytes));
        HS_HIP(hipDeviceSynchronize());
        g_scratch[device] = p;
      }
      g_prepared.push_back(device);
    }
  }
  hs_context *ctx = new (std::nothrow) hs_context();
  if (!ctx) return fail(HS_ERR_OUT_OF_MEMORY, "host allocation failed");
  ctx->device = device;
  if (const char *env = getenv("HS_ROW_KERNEL_MIN_ROWS")) ctx->row_min_rows = atoi(env);
  if (const char *env = getenv("HS_ROW_SPLIT")) ctx->row_split = atoi(env);
  if (const char *env = getenv("HS_LMHEAD_FUSE")) ctx->fuse = atoi(env);
  e = hipEventCreateWithFlags(&ctx->plan_done, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->done_ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->na_upload_ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipHostMalloc(&ctx->na_staging, na::kPlansBytes + na::kListsBytes);
  if (e == hipSuccess) {
    ctx->na_last = new (std::nothrow) hs_sample_config[na::kMaxRows];
    if (!ctx->na_last) e = hipErrorOutOfMemory;
  }
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    hs_context_destroy(ctx);
    return fail(HS_ERR_HIP, "context setup failed: %s", hipGetErrorString(e));
  }
  *out = ctx;
  return HS_OK;
}

int hs_context_set_timing(hs_context *ctx, int enable) {
  HS_LOCK(ctx);
  ctx->timing = enable != 0;
  return HS_OK;
}

int hs_context_kernel_times(hs_context *ctx, double *ms, int32_t count, int64_t *calls) {
  HS_LOCK(ctx);
  if (count < 0 || (count > 0 && !ms)) return fail(HS_ERR_INVALID_ARGUMENT, "bad output array");
  DeviceGuard guard(ctx->device);
  for (const hs_context::TimedCall &tc : ctx->timed) {
    for (int k = 0; k < hs::kTimedKernels; ++k) {
      if (!(tc.mask >> k & 1u)) continue;
      float t = 0;
      HS_HIP(hipEventSynchronize(tc.ev[2 * k + 1]));
      HS_HIP(hipEventElapsedTime(&t, tc.ev[2 * k], tc.ev[2 * k + 1]));
      ctx->kernel_ms[k] += t;
    }
    ++ctx->timed_calls;
  }
  for (const hs_context::TimedCall &tc : ctx->timed)
    for (int i = 0; i < 2 * hs::kTimedKernels; ++i)
      if (tc.mask >> (i / 2) & 1u) ctx->ev_free.push_back(tc.ev[i]);
  ctx->timed.clear();
  for (int k = 0; k < count; ++k) ms[k] = k < hs::kTimedKernels ? ctx->kernel_ms[k] : 0.0;
  if (calls) *calls = ctx->timed_calls;
  for (int k = 0; k < hs::kTimedKernels; ++k) ctx->kernel_ms[k] = 0;
  ctx->timed_calls = 0;
  return HS_OK;
}

int hs_context_destroy(hs_context *ctx) {
  if (!ctx) return HS_OK;
  {
    DeviceGuard guard(ctx->device);
    (void)hipDeviceSynchronize();
    for (hipEvent_t x : ctx->ev_free) (void)hipEventDestroy(x);
    for (const hs_context::TimedCall &tc : ctx->timed)
      for (int i = 0; i < 2 * hs::kTimedKernels; ++i)
        if (tc.mask >> (i / 2) & 1u) (void)hipEventDestroy(tc.ev[i]);
    ctx->plans.release();
    ctx->cand.release();
    ctx->cand_count.release();
    ctx->info.release();
    ctx->split_list.release();
    ctx->split_meta.release();
    ctx->split_cnt.release();
    ctx->gemv_part.release();
    ctx->gemv_cnt.release();
    ctx->gemv_rot.release();
    ctx->large_retry.release();
    ctx->large_replay.release();
    ctx->replay_slots.release();
    ctx->h_logits.release();
    ctx->h_small.release();
    ctx->h_tok.release();
    ctx->h_pin.release();
    if (ctx->plan_staging) (void)hipHostFree(ctx->plan_staging);
    if (ctx->plan_done) (void)hipEventDestroy(ctx->plan_done);
    if (ctx->done_ev) (void)hipEventDestroy(ctx->done_ev);
    if (ctx->na_upload_ev) (void)hipEventDestroy(ctx->na_upload_ev);
    if (ctx->na_staging) (void)hipHostFree(ctx->na_staging);
    delete[] ctx->na_last;
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
  return HS_OK;
}

int hs_sample_batch_device_ex(hs_context *ctx, float *d_logits, int32_t rows, int64_t row_stride,
                              int32_t vocab, const int32_t *d_hist_ids,
                              const int64_t *d_hist_offsets, const hs_sample_config *configs,
                              const double *d_uniforms, int32_t *d_tokens, int32_t cand_stride,
                              int32_t *d_cand_ids, float *d_cand_probs, int32_t *d_cand_count,
                              int32_t *d_cutoff, uint32_t *d_row_flags, void *stream) {
  HS_LOCK(ctx);
  return sample_device(ctx, d_logits, rows, row_stride, vocab, d_hist_ids, d_hist_offsets, configs,
                       d_uniforms, d_tokens, cand_stride, d_cand_ids, d_cand_probs, d_cand_count,
                       d_cutoff, d_row_flags, static_cast<hipStream_t>(stream));
}

int hs_sample_batch_device(hs_context *ctx, float *d_logits, int32_t rows, int64_t row_stride,
                           int32_t vocab, const int32_t *d_hist_ids,
                           const int64_t *d_hist_offsets, const hs_sample_config *configs,
                           const double *d_uniforms, int32_t *d_tokens, void *stream) {
  HS_LOCK(ctx);
  return sample_device(ctx, d_logits, rows, row_stride, vocab, d_hist_ids, d_hist_offsets, configs,
                       d_uniforms, d_tokens, 0, nullptr, nullptr, nullptr, nullptr, nullptr,
                       static_cast<hipStream_t>(stream));
}

int hs_sample_batch_device_noalloc(hs_context *ctx, float *d_logits, int32_t rows,
                                   int64_t row_stride, int32_t vocab, const int32_t *d_hist_ids,
                                   const int64_t *d_hist_offsets, const hs_sample_config *configs,
                                   const double *d_uniforms, int32_t *d_tokens, void *stream) {
  HS_LOCK(ctx);
  return sample_device_noalloc(ctx, d_logits, rows, row_stride, vocab, d_hist_ids, d_hist_offsets,
                               configs, d_uniforms, d_tokens, static_cast<hipStream_t>(stream));
}

int hs_argmax_device(hs_context *ctx, const float *d_logits, int32_t rows, int64_t row_stride,
                     int32_t vocab, int32_t *d_tokens, void *stream) {
  HS_LOCK(ctx);
  return argmax_device(ctx, d_logits, rows, row_stride, vocab, d_tokens,
                       static_cast<hipStream_t>(stream));
}

namespace {
hs_weights raw_weights(int32_t K, const void *d_w, int32_t w_type, int32_t N) {
  hs_weights w;
  memset(&w, 0, sizeof w);
  w.type = w_type;
  w.rows = N;
  w.cols = K;
  w.data = d_w;
  return w;
}
}  // namespace

int hs_gemv_device(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx, int32_t K,
                   const void *d_w, int32_t w_type, int32_t N, float *d_y, int64_t ldy,
                   void *stream) {
  HS_LOCK(ctx);
  if (hs::tern_quant_bytes(w_type) > 0)
    return fail(HS_ERR_INVALID_ARGUMENT, "weight type %d is planar: use hs_gemv_device_ex", w_type);
  const hs_weights w = raw_weights(K, d_w, w_type, N);
  return gemv_device(ctx, d_x, M, ldx, &w, d_y, ldy, static_cast<hipStream_t>(stream));
}

int hs_gemv_device_ex(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx,
                      const hs_weights *w, float *d_y, int64_t ldy, void *stream) {
  HS_LOCK(ctx);
  return gemv_device(ctx, d_x, M, ldx, w, d_y, ldy, static_cast<hipStream_t>(stream));
}

namespace {

// The lm_head GEMV and the sampler on its M rows: one launch of the planar,
// Q4_K or Q6_K GEMV that samples its own rows when every row is greedy or takes
// k <= 64 candidates with at most the repetition penalty (and the vocabulary
// fits its per-wave record); otherwise the GEMV, then
// hs_sample_batch_device.  Either way the logits hold the penalised values
// afterwards.  By default the one launch is taken only when every row is
// greedy: with sampling rows its merge (the last workgroup of the row) takes
// about as long as the sampler's own launch, or longer.
int lm_head_sample(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx, const hs_weights *w,
                   float *d_logits, int64_t ldl, const int32_t *d_hist_ids,
                   const int64_t *d_hist_offsets, const hs_sample_config *configs,
                   const double *d_uniforms, int32_t *d_tokens, hipStream_t st) {
  if (!ctx) return fail(HS_ERR_INVALID_ARGUMENT, "null context");
  if (!w) return fail(HS_ERR_INVALID_ARGUMENT, "null weights");
  const bool tern = hs::tern_quant_bytes(w->type) > 0;
  // sampling rows fuse into the planar, Q4_K and Q6_K GEMVs only (their
  // 16-row tiles); the vector-unit GEMVs fuse greedy rows only when asked
  // (HS_LMHEAD_FUSE=2): their argmax launch measured 2.7 us (no penalty) to
  // 9 us (repetition penalty) slower than the GEMV and the argmax launch
  const bool sample_ok = tern || w->type == hs::kW_Q6_K || w->type == hs::kW_Q4_K;
  bool fused = ctx->fuse && (sample_ok || ctx->fuse >= 2) && M > 0 && w->rows > 0 && configs &&
               d_uniforms && d_tokens && (d_hist_ids == nullptr) == (d_hist_offsets == nullptr);
  std::vector<hs::RowPlan> plans;
  Routing rt;
  if (fused) {
    try {
      int rc = build_plans(configs, M, w->rows, ctx->row_min_rows, plans, rt);
      if (rc) return rc;
    } catch (const std::bad_alloc &) {
      return fail(HS_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    for (const hs::RowPlan &p : plans) {
      if ((p.mode != hs::kModeGreedy && p.mode != hs::kModeSmall) || (p.pen & hs::kPenPF))
        fused = false;
      if ((ctx->fuse < 2 || !sample_ok) && p.mode != hs::kModeGreedy) fused = false;
    }
  }
  // every row greedy: the GEMV keeps the argmax alone
  bool greedy = fused;
  for (const hs::RowPlan &p : plans) greedy = greedy && p.mode == hs::kModeGreedy;
  if (fused) {
    DeviceGuard guard(ctx->device);
    int rc = enter_stream(ctx, st);
    if (rc) return rc;
    hs::GemvArgs g;
    bool skip = false;
    rc = gemv_setup(ctx, d_x, M, ldx, w, d_logits, ldl, st, g, &skip);
    if (rc) return rc;
    const int blocks = skip     ? 0
                       : greedy ? hs::argmax_fused_grid(g)
                       : tern   ? hs::tern_sample_grid(g)
                                : hs::kq_sample_grid(g);
    if (blocks > 0) {
      const size_t nwv = greedy ? 0 : (size_t)M * blocks * hs::fuse_waves_per_block(w->type);
      if (!greedy) {
        HS_HIP(ctx->fuse_pool.ensure(nwv * (2 * sizeof(unsigned long long) +
                                            hs::kFuseTileWords * sizeof(int32_t))));
        // histograms: zero between calls (each is cleared by the workgroup that reads it)
        rc = ensure_zeroed(ctx->fuse_hist, (size_t)M * hs::kFuseHist * sizeof(uint32_t), st);
        if (rc) return rc;
      }
      // counters: zero between calls (each is reset by the workgroup that counts last)
      rc = ensure_zeroed(ctx->fuse_rows, (size_t)M * sizeof(hs::FuseRow), st);
      if (rc) return rc;
      rc = upload_plans(ctx, plans, rt, w->rows, st);
      if (rc) return rc;
      hs::FuseArgs f;
      f.plans = static_cast<const hs::RowPlan *>(ctx->plans.p);
      f.hist_ids = d_hist_ids;
      f.hist_off = d_hist_offsets;
      f.uniforms = d_uniforms;
      f.tokens = d_tokens;
      f.rows = static_cast<hs::FuseRow *>(ctx->fuse_rows.p);
      f.wtop = greedy ? nullptr : static_cast<unsigned long long *>(ctx->fuse_pool.p);
      f.wtiles = greedy ? nullptr : reinterpret_cast<int32_t *>(f.wtop + 2 * nwv);
      f.hist = greedy ? nullptr : static_cast<uint32_t *>(ctx->fuse_hist.p);
      f.blocks = blocks;
      hipEvent_t *ev = nullptr;
      rc = timed_slot(ctx, hs::kGemvTimedSlot, &ev);
      if (rc) return rc;
      const hipError_t e = greedy ? hs::launch_argmax_fused(g, f, st, ev, ctx->done_ev)
                           : tern ? hs::launch_tern_sample(g, f, st, ev, ctx->done_ev)
                                  : hs::launch_kq_sample(g, f, st, ev, ctx->done_ev);
      if (e != hipSuccess) {
        (void)leave_stream(ctx, st, false);
        return fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
      }
      return leave_stream(ctx, st, ev == nullptr);
    }
    if (g.x != d_x) (void)leave_stream(ctx, st, false);   // the rotation was enqueued
  }
  int rc = gemv_device(ctx, d_x, M, ldx, w, d_logits, ldl, st);
  if (rc) return rc;
  return sample_device(ctx, d_logits, M, ldl, w->rows, d_hist_ids, d_hist_offsets, configs,
                       d_uniforms, d_tokens, 0, nullptr, nullptr, nullptr, nullptr, nullptr, st);
}

}  // namespace

int hs_lm_head_sample_device(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx, int32_t K,
                             const void *d_w, int32_t w_type, int32_t N, float *d_logits,
                             int64_t ldl, const int32_t *d_hist_ids, const int64_t *d_hist_offsets,
                             const hs_sample_config *configs, const double *d_uniforms,
                             int32_t *d_tokens, void *stream) {
  HS_LOCK(ctx);
  if (hs::tern_quant_bytes(w_type) > 0)
    return fail(HS_ERR_INVALID_ARGUMENT, "weight type %d is planar: use hs_lm_head_sample_device_ex",
                w_type);
  const hs_weights w = raw_weights(K, d_w, w_type, N);
  return lm_head_sample(ctx, d_x, M, ldx, &w, d_logits, ldl, d_hist_ids, d_hist_offsets, configs,
                        d_uniforms, d_tokens, static_cast<hipStream_t>(stream));
}

int hs_lm_head_sample_device_ex(hs_context *ctx, const float *d_x, int32_t M, int64_t ldx,
                                const hs_weights *w, float *d_logits, int64_t ldl,
                                const int32_t *d_hist_ids, const int64_t *d_hist_offsets,
                                const hs_sample_config *configs, const double *d_uniforms,
                                int32_t *d_tokens, void *stream) {
  HS_LOCK(ctx);
  return lm_head_sample(ctx, d_x, M, ldx, w, d_logits, ldl, d_hist_ids, d_hist_offsets, configs,
                        d_uniforms, d_tokens, static_cast<hipStream_t>(stream));
}

// src/engine.ts:80-175 (createBlockSplitter): GGUF blocks of Q1_0 ([d][16 B
// signs]), PQ2_0 ([d][32 B codes]) or PTQ1_0 ([24 B qs][2 B qh][d]) into the
// planar quants and binary16 scales the GEMV reads.
int hs_split_blocks(int32_t type, const void *blocks, int64_t n_blocks, void *quants,
                    void *scales16) {
  const int qb = hs::tern_quant_bytes(type);
  if (qb == 0) return fail(HS_ERR_INVALID_ARGUMENT, "type %d has no planar form", type);
  if (n_blocks < 0) return fail(HS_ERR_INVALID_ARGUMENT, "n_blocks must be >= 0");
  if (n_blocks > 0 && (!blocks || !quants || !scales16))
    return fail(HS_ERR_INVALID_ARGUMENT, "blocks, quants and scales16 must not be null");
  const int bb = qb + 2;
  const uint8_t *src = static_cast<const uint8_t *>(blocks);
  uint8_t *q = static_cast<uint8_t *>(quants);
  uint8_t *sc = static_cast<uint8_t *>(scales16);
  const bool scale_last = type == hs::kW_PTQ1_0;
  for (int64_t b = 0; b < n_blocks; ++b) {
    const uint8_t *blk = src + b * bb;
    memcpy(q + b * qb, scale_last ? blk : blk + 2, (size_t)qb);
    memcpy(sc + b * 2, scale_last ? blk + qb : blk, 2);
  }
  return HS_OK;
}

// src/engine.ts:1626-1644 (one step of the decode loop) with the token
// history kept on the GPU.
int hs_decode_step_device(hs_context *ctx, float *d_logits, int32_t rows, int64_t row_stride,
                          int32_t vocab, int32_t *d_ring, int64_t ring_cap, int64_t *d_len,
                          int32_t *d_done, const int32_t *d_stop_ids, int32_t n_stop,
                          const hs_sample_config *configs, const double *d_uniforms,
                          int32_t *d_tokens, void *stream) {
  HS_LOCK(ctx);
  if (rows < 0) return fail(HS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %d)", rows);
  if (rows == 0) return HS_OK;
  if (!d_ring || !d_len || !d_done)
    return fail(HS_ERR_INVALID_ARGUMENT, "ring, len and done must not be null");
  if (ring_cap < 128 || ring_cap > (int64_t(1) << 29))
    return fail(HS_ERR_INVALID_ARGUMENT, "ring_cap must be in [128, 2^29] (got %lld)",
                (long long)ring_cap);
  if (n_stop < 0 || n_stop > hs::kMaxStopIds)
    return fail(HS_ERR_INVALID_ARGUMENT, "n_stop must be in [0, %d] (got %d)", hs::kMaxStopIds,
                n_stop);
  if (n_stop > 0 && !d_stop_ids) return fail(HS_ERR_INVALID_ARGUMENT, "stop ids must not be null");
  hs::DecodeArgs d;
  d.tokens = d_tokens;
  d.ring = d_ring;
  d.cap = ring_cap;
  d.len = d_len;
  d.done = d_done;
  d.stop_ids = d_stop_ids;
  d.n_stop = n_stop;
  d.rows = rows;
  // the bookkeeping runs where each row's token is written
  return sample_device(ctx, d_logits, rows, row_stride, vocab, d_ring, nullptr, configs, d_uniforms,
                       d_tokens, 0, nullptr, nullptr, nullptr, nullptr, nullptr,
                       static_cast<hipStream_t>(stream), d_len, ring_cap, &d);
}

int hs_argmax(hs_context *ctx, const float *logits, int32_t rows, int64_t row_stride,
              int32_t vocab, int32_t *tokens_out) {
  HS_LOCK(ctx);
  if (rows < 0) return fail(HS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %d)", rows);
  if (rows == 0) return HS_OK;
  if (!tokens_out) return fail(HS_ERR_INVALID_ARGUMENT, "tokens_out must not be null");
  if (vocab <= 0) {
    for (int r = 0; r < rows; ++r) tokens_out[r] = 0;
    return HS_OK;
  }
  if (!logits) return fail(HS_ERR_INVALID_ARGUMENT, "logits must not be null");
  if (row_stride < vocab)
    return fail(HS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  if (vocab > hs::kArgmaxMaxVocab)
    return fail(HS_ERR_UNSUPPORTED, "vocab %d above %d", vocab, hs::kArgmaxMaxVocab);
  DeviceGuard guard(ctx->device);
  hipStream_t st = ctx->stream;
  const size_t lbytes = sizeof(float) * ((size_t)(rows - 1) * (size_t)row_stride + (size_t)vocab);
  const bool stage = lbytes <= kPinLogitsMax;
  const size_t o_tok = stage ? pin_align(lbytes) : 0;
  HS_HIP(ctx->h_logits.ensure(lbytes));
  HS_HIP(ctx->h_tok.ensure(sizeof(int32_t) * rows));
  HS_HIP(ctx->h_pin.ensure(o_tok + sizeof(int32_t) * rows));
  char *pin = static_cast<char *>(ctx->h_pin.p);
  if (stage) memcpy(pin, logits, lbytes);
  HS_HIP(hipMemcpyAsync(ctx->h_logits.p, stage ? static_cast<const void *>(pin) : logits, lbytes,
                        hipMemcpyHostToDevice, st));
  int rc = argmax_device(ctx, static_cast<float *>(ctx->h_logits.p), rows, row_stride, vocab,
                         static_cast<int32_t *>(ctx->h_tok.p), st);
  if (rc) {
    (void)hipStreamSynchronize(st);
    return rc;
  }
  const hipError_t e = inject_failure() ? hipErrorOutOfMemory
                                        : hipMemcpyAsync(pin + o_tok, ctx->h_tok.p,
                                                         sizeof(int32_t) * rows,
                                                         hipMemcpyDeviceToHost, st);
  const hipError_t es = hipStreamSynchronize(st);   // the staging is free again either way
  if (e != hipSuccess) return fail(HS_ERR_HIP, "token copy failed: %s", hipGetErrorString(e));
  if (es != hipSuccess) return fail(HS_ERR_HIP, "hipStreamSynchronize failed: %s", hipGetErrorString(es));
  memcpy(tokens_out, pin + o_tok, sizeof(int32_t) * rows);
  return HS_OK;
}

int hs_sample_logits_batch(hs_context *ctx, float *logits, int32_t rows, int64_t row_stride,
                           int32_t vocab, const int32_t *hist_ids, const int64_t *hist_offsets,
                           const hs_sample_config *configs, const double *uniforms,
                           int32_t *tokens_out) {
  HS_LOCK(ctx);
  if (rows < 0) return fail(HS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %d)", rows);
  if (rows == 0) return HS_OK;
  if (!configs || !uniforms || !tokens_out)
    return fail(HS_ERR_INVALID_ARGUMENT, "configs, uniforms and tokens_out must not be null");
  if ((hist_ids == nullptr) != (hist_offsets == nullptr))
    return fail(HS_ERR_INVALID_ARGUMENT, "history ids and offsets must both be given or both null");
  if (vocab <= 0) {
    for (int r = 0; r < rows; ++r) tokens_out[r] = 0;
    return HS_OK;
  }
  if (!logits) return fail(HS_ERR_INVALID_ARGUMENT, "logits must not be null");
  if (row_stride < vocab)
    return fail(HS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  int64_t hist_total = 0;
  if (hist_offsets) {
    if (hist_offsets[0] != 0)
      return fail(HS_ERR_INVALID_ARGUMENT, "hist_offsets[0] must be 0");
    for (int r = 0; r < rows; ++r)
      if (hist_offsets[r + 1] < hist_offsets[r])
        return fail(HS_ERR_INVALID_ARGUMENT, "hist_offsets must be non-decreasing (row %d)", r);
    hist_total = hist_offsets[rows];
  }
  DeviceGuard guard(ctx->device);
  hipStream_t st = ctx->stream;
  const size_t lbytes = sizeof(float) * ((size_t)(rows - 1) * (size_t)row_stride + (size_t)vocab);
  // The reference writes the penalised values back (src/sampler.ts:30).
  // Only history ids change: the last 128 of a row for the repetition
  // penalty, all of them with presence / frequency.  Their offsets are listed
  // here, and a kernel gathers those entries (and the tokens) into the pinned
  // buffer after sampling: no copy of the whole block back.
  try {
    ctx->gidx.clear();
    for (int r = 0; r < rows && hist_offsets; ++r) {
      const hs_sample_config &c = configs[r];
      const bool rep = c.repetition_penalty != 1.0;
      const bool pf = c.presence_penalty != 0.0 || c.frequency_penalty != 0.0;
      if (!(rep || pf)) continue;
      const int64_t h1 = hist_offsets[r + 1];
      const int64_t h0 = pf ? hist_offsets[r] : std::max(hist_offsets[r], h1 - 128);
      for (int64_t j = h0; j < h1; ++j) {
        const int32_t id = hist_ids[j];
        if (id >= 0 && id < vocab) ctx->gidx.push_back((int64_t)r * row_stride + id);
      }
    }
  } catch (const std::bad_alloc &) {
    return fail(HS_ERR_OUT_OF_MEMORY, "host allocation failed");
  }
  const int64_t ng = (int64_t)ctx->gidx.size();
  bool zero_copy = lbytes <= kZeroCopyMax;
  for (int r = 0; r < rows && zero_copy; ++r)
    zero_copy = plan_row(configs[r], vocab).mode != hs::kModeLarge;
  if (zero_copy) return sample_host_zero_copy(ctx, logits, lbytes, rows, row_stride, vocab, hist_ids,
                                              hist_offsets, hist_total, configs, uniforms,
                                              tokens_out);
  // pinned layout: [logits (when staged)] [uniforms | offsets | history ids]
  // [gathered offsets] [gathered values] [tokens]; the device copy of the
  // middle part has the same layout, so one copy moves it
  const bool stage = lbytes <= kPinLogitsMax;
  const size_t o_small = stage ? pin_align(lbytes) : 0;
  const size_t s_u = sizeof(double) * rows;
  const size_t s_off = hist_offsets ? sizeof(int64_t) * (size_t)(rows + 1) : 0;
  const size_t s_hist = sizeof(int32_t) * (size_t)hist_total;
  const size_t r_off = pin_align(s_u), r_hist = r_off + pin_align(s_off);
  const size_t small_bytes = r_hist + s_hist;
  const size_t o_gidx = o_small + pin_align(small_bytes);
  const size_t o_gval = o_gidx + pin_align(sizeof(int64_t) * (size_t)ng);
  const size_t o_tok = o_gval + pin_align(sizeof(float) * (size_t)ng);
  HS_HIP(ctx->h_logits.ensure(lbytes));
  HS_HIP(ctx->h_small.ensure(small_bytes));
  HS_HIP(ctx->h_tok.ensure(sizeof(int32_t) * rows));
  HS_HIP(ctx->h_pin.ensure(o_tok + sizeof(int32_t) * rows));
  char *pin = static_cast<char *>(ctx->h_pin.p);
  char *small = pin + o_small;
  if (stage) memcpy(pin, logits, lbytes);
  memcpy(small, uniforms, s_u);
  if (hist_offsets) {
    memcpy(small + r_off, hist_offsets, s_off);
    if (hist_total > 0) memcpy(small + r_hist, hist_ids, s_hist);
  }
  if (ng > 0) memcpy(pin + o_gidx, ctx->gidx.data(), sizeof(int64_t) * (size_t)ng);
  // from the first copy on, every return waits for the stream first: the
  // pinned buffer must not be refilled while a copy still reads it
  auto bail = [&](int rc) {
    (void)hipStreamSynchronize(st);
    return rc;
  };
  HS_HIP(hipMemcpyAsync(ctx->h_logits.p, stage ? static_cast<const void *>(pin) : logits, lbytes,
                        hipMemcpyHostToDevice, st));
  hipError_t e = inject_failure() ? hipErrorOutOfMemory
                                  : hipMemcpyAsync(ctx->h_small.p, small, small_bytes,
                                                   hipMemcpyHostToDevice, st);
  if (e != hipSuccess)
    return bail(fail(HS_ERR_HIP, "input copy failed: %s", hipGetErrorString(e)));
  char *dsmall = static_cast<char *>(ctx->h_small.p);
  const int32_t *d_ids = hist_offsets ? reinterpret_cast<const int32_t *>(dsmall + r_hist) : nullptr;
  const int64_t *d_off = hist_offsets ? reinterpret_cast<const int64_t *>(dsmall + r_off) : nullptr;
  int rc = sample_device(ctx, static_cast<float *>(ctx->h_logits.p), rows, row_stride, vocab, d_ids,
                         d_off, configs, reinterpret_cast<const double *>(dsmall),
                         static_cast<int32_t *>(ctx->h_tok.p), 0, nullptr, nullptr, nullptr, nullptr,
                         nullptr, st);
  if (rc) return bail(rc);
  e = inject_failure() ? hipErrorOutOfMemory
                       : hs::launch_gather_out(static_cast<const float *>(ctx->h_logits.p),
                                               reinterpret_cast<const int64_t *>(pin + o_gidx),
                                               reinterpret_cast<float *>(pin + o_gval), ng,
                                               static_cast<const int32_t *>(ctx->h_tok.p),
                                               reinterpret_cast<int32_t *>(pin + o_tok), rows, st);
  if (e != hipSuccess)
    return bail(fail(HS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e)));
  HS_HIP(hipStreamSynchronize(st));
  memcpy(tokens_out, pin + o_tok, sizeof(int32_t) * rows);
  const float *gval = reinterpret_cast<const float *>(pin + o_gval);
  for (int64_t i = 0; i < ng; ++i) logits[ctx->gidx[i]] = gval[i];
  for (int r = 0; r < rows; ++r)
    if (tokens_out[r] < 0)
      return fail(HS_ERR_UNSUPPORTED,
                  "row %d: top-k above %d with equal logits at the drawn position; the "
                  "reference orders them by its slot history, which this build replays up to "
                  "that top-k only", r, hs::kReplayDevMaxK);
  return HS_OK;
}

int hs_sample_logits(hs_context *ctx, float *logits, int32_t vocab, const int32_t *history,
                     int64_t history_len, const hs_sample_config *config, double uniform,
                     int32_t *token_out) {
  if (history_len < 0) return fail(HS_ERR_INVALID_ARGUMENT, "history_len must be >= 0");
  if (history_len > 0 && !history)
    return fail(HS_ERR_INVALID_ARGUMENT, "history must not be null when history_len > 0");
  const int64_t off[2] = {0, history_len};
  return hs_sample_logits_batch(ctx, logits, 1, vocab > 0 ? vocab : 1, vocab,
                                history_len > 0 ? history : nullptr,
                                history_len > 0 ? off : nullptr, config, &uniform, token_out);
}

}  // extern "C"
