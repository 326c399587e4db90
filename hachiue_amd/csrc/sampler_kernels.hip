// gfx950 kernels of the logits-to-token sampler.
//
// Semantics follow hachiue's sampleLogits (src/sampler.ts:12-118): logits are
// binary32, all arithmetic after the load is binary64 and results are rounded
// to binary32 exactly where the reference stores into a Float32Array.  This
// file must be compiled with -ffp-contract=off so no multiply-add is fused.
//
// Kernels of one call (rows are routed by the host):
//   pen_kernel       rows with presence / frequency penalties, one
//                    1024-thread workgroup per row: counts the history's
//                    distinct ids in an LDS hash table and applies the
//                    repetition penalty (last 128 ids) and the extension in
//                    place.
//   row_kernel       greedy rows and rows with k <= 64, one 1024-thread
//                    workgroup per row (the hot path).  The row streams from
//                    HBM in rounds of 32768 logits, two rounds in registers.
//                    Round 0 fixes a lower bound of the row's k-th largest
//                    value (the exact k-th largest of the 1024 lane maxima);
//                    every logit at or above it is appended to an LDS
//                    candidate list.  The workgroup then ranks, samples and
//                    writes the row itself: one HBM pass, one launch.  Small
//                    batches split each row over up to 16 workgroups; the
//                    last part to finish merges the parts' top-64 lists.
//   mid_kernel       rows with 64 < k <= 1024 (and, in calls that launch it,
//                    the k <= 64 rows): the row kernel's stream with the
//                    bound from an LDS key histogram.
//   chunk_kernel     rows of vocabularies above 512K (and calls below the
//                    row kernel's minimum batch), grid rows*S, 256 threads: a
//                    chunk of 16384 logits in registers, exact chunk k-th
//                    largest by block radix select, candidates to a per-row
//                    list.
//   finalize_kernel  one workgroup per chunk-kernel row: exact select over the
//                    row's candidates, then the shared row completion.
//   large_kernel     rows with k > 1024: one 1024-thread workgroup per row,
//                    several passes (radix select of the k-th value, softmax
//                    normaliser, probability-mass histogram, positions located
//                    by narrowing one bucket).
// Row completion (finish_row): equal-value groups make the reference's order
// depend on its slot history (src/sampler.ts:55-69); when such a group can
// change the result, the exact replace-min scan is replayed over the row.
#include "sampler_internal.h"

#include <hip/hip_ext.h>

#include <float.h>
#include <type_traits>
#include <math.h>

#include "hachiue_sampler.h"
#include "blk_gemv.h"
#include "kq_gemv.h"
#include "tern_gemv.h"

namespace hs {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- keys

// Order-preserving key of a binary32 value: larger value <=> larger key.
// -0 shares the key of +0 (the reference's comparisons treat them as equal);
// NaN and -Infinity, which never enter the reference's top-k (`v > minVal` is
// false for them, src/sampler.ts:57), map to 0.
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t u = __float_as_uint(f);
  u = (u == 0x80000000u) ? 0u : u;
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (f > -INFINITY) ? k : 0u;
}

__device__ __forceinline__ float key2f(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

// Float threshold x with {v : v >= x} == {v : f2key(v) >= X} for a key X of a
// real value (X >= 1; X at or below the key of -FLT_MAX keeps every finite).
__device__ __forceinline__ float key_floor(uint32_t X) {
  return X <= 0x00800000u ? -FLT_MAX : key2f(X);
}

// Candidate composite: key in the high word, ~index in the low word, so a
// descending sort orders by value descending and index ascending.
__device__ __forceinline__ unsigned long long pack_cand(uint32_t key, uint32_t idx) {
  return ((unsigned long long)key << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t cand_key(unsigned long long c) { return (uint32_t)(c >> 32); }
__device__ __forceinline__ uint32_t cand_idx(unsigned long long c) { return 0xFFFFFFFFu - (uint32_t)c; }

// Wave-uniform read of memory the kernel never writes, through the scalar
// cache (constant address space): it completes independently of the vector
// loads queued before it.
template <typename T>
__device__ __forceinline__ T load_scalar(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// ---------------------------------------------------------------- wave helpers

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

__device__ __forceinline__ uint32_t lanes_below(unsigned long long mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t readlane_u32(uint32_t x, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, lane);
}
__device__ __forceinline__ float readlane_f32(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
__device__ __forceinline__ double readlane_f64(double x, int lane) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(x);
  const uint32_t lo = readlane_u32((uint32_t)b, lane), hi = readlane_u32((uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Exact k-th largest of one key per lane (1 <= k <= 64) by a binary search
// over the key bits: the largest t with at least k lanes holding a key >= t.
// Returns 0 when fewer than k lanes hold a non-zero key.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t key, int k) {
  if (__popcll(__ballot(key != 0u)) < k) return 0u;
  uint32_t t = 0;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = t | (1u << b);
    if (__popcll(__ballot(key >= c)) >= k) t = c;
  }
  return t;
}

__device__ __forceinline__ unsigned long long wave_sort_desc64(unsigned long long x) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const unsigned long long y = __shfl_xor(x, stride);
      const bool lower = (lane & stride) == 0;
      const bool desc = (lane & size) == 0;
      x = (lower == desc) ? (x > y ? x : y) : (x < y ? x : y);
    }
  }
  return x;
}

__device__ __forceinline__ unsigned long long wave_max64(unsigned long long x) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const unsigned long long y = __shfl_xor(x, m);
    x = x > y ? x : y;
  }
  return x;
}

// ---------------------------------------------------------------- block helpers

// Inclusive prefix sum over the NT threads of the block (wsum: NT/64 words).
// Contains one barrier; reuses of wsum must be separated by another barrier.
template <int NT>
__device__ __forceinline__ uint32_t block_scan_incl(uint32_t x, uint32_t *wsum) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  uint32_t add = 0;
  for (int w = 0; w < wave; ++w) add += wsum[w];
  return x + add;
}

struct SelectSmem {
  uint32_t hist[256];
  uint32_t wsum[16];
  int32_t digit, above, total;
};

// Inclusive prefix sum across a wave64 with DPP row shifts and row
// broadcasts (no LDS traffic).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t x) {
  // row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false);
  return x;
}

// Inclusive prefix sum of one binary64 value per lane over the wave (DPP row
// shifts and row broadcasts on both halves of the value).
__device__ __forceinline__ double wave_scan_incl_f64(double x) {
  // row_shr:n = 0x110 + n (bound_ctrl: 0 where the source lane is outside the
  // row), row_bcast:15 = 0x142 into rows 1 and 3, row_bcast:31 = 0x143 into
  // rows 2 and 3 (other rows keep 0)
#define HS_DPP_ADD(ctrl, rmask, bc)                                                        \
  {                                                                                        \
    const unsigned long long b = (unsigned long long)__double_as_longlong(x);              \
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, ctrl,   \
                                                               rmask, 0xF, bc);            \
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), \
                                                               ctrl, rmask, 0xF, bc);      \
    x += __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));           \
  }
  HS_DPP_ADD(0x111, 0xF, true)
  HS_DPP_ADD(0x112, 0xF, true)
  HS_DPP_ADD(0x114, 0xF, true)
  HS_DPP_ADD(0x118, 0xF, true)
  HS_DPP_ADD(0x142, 0xA, false)
  HS_DPP_ADD(0x143, 0xC, false)
#undef HS_DPP_ADD
  return x;
}

// Exact k-th largest key of a block-wide multiset, four 8-bit digit passes.
// All threads add their keys to a 256-bin LDS histogram; wave 0 alone finds
// the digit (bins scanned from the top, four per lane) and clears the bins
// for the next pass: two barriers per pass.  `hist_pass(shift, prefix, pass)`
// adds this thread's keys (see hist_add).  Returns T, or 0 when fewer than k
// keys participate; *total receives the participant count.
template <int NT, typename HistPass>
__device__ __forceinline__ uint32_t block_select_fast(int k, HistPass hist_pass, SelectSmem &sm,
                                                      int *total) {
  const int tid = threadIdx.x;
  if (tid < 256) sm.hist[tid] = 0;
  __syncthreads();
  uint32_t prefix = 0;
  int rem = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist_pass(shift, prefix, pass);
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 255-4l .. 252-4l (descending digit order)
      uint32_t c[4], part = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = sm.hist[255 - 4 * tid - i];
        sm.hist[255 - 4 * tid - i] = 0;
        part += c[i];
      }
      const uint32_t incl = wave_scan_incl(part);
      if (pass == 0 && tid == 63) sm.total = (int)incl;
      uint32_t run = incl - part;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (run < (uint32_t)rem && run + c[i] >= (uint32_t)rem) {
          sm.digit = 255 - 4 * tid - i;
          sm.above = (int)run;
        }
        run += c[i];
      }
    }
    __syncthreads();
    if (pass == 0) {
      *total = sm.total;
      if (sm.total < k) return 0u;
    }
    prefix |= (uint32_t)sm.digit << shift;
    rem -= sm.above;
  }
  return prefix;
}

// Exact k-th largest key of a block-wide multiset: four 8-bit digit passes
// over a 256-bin LDS histogram.  `hist_pass(shift, prefix, pass)` adds this
// thread's keys (see hist_add).  Returns T, or 0 when fewer than k keys
// participate; *total receives the participant count.
template <int NT, typename HistPass>
__device__ __forceinline__ uint32_t block_select(int k, HistPass hist_pass, SelectSmem &sm, int *total) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0;
  int rem = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) sm.hist[tid] = 0;
    __syncthreads();
    hist_pass(shift, prefix, pass);
    __syncthreads();
    const uint32_t c = tid < 256 ? sm.hist[255 - tid] : 0u;
    const uint32_t incl = block_scan_incl<NT>(c, sm.wsum);
    if (pass == 0 && tid == 255) sm.total = (int)incl;
    if (tid < 256 && incl >= (uint32_t)rem && incl - c < (uint32_t)rem) {
      sm.digit = 255 - tid;
      sm.above = (int)(incl - c);
    }
    __syncthreads();
    if (pass == 0) {
      *total = sm.total;
      if (sm.total < k) return 0u;
    }
    prefix |= (uint32_t)sm.digit << shift;
    rem -= sm.above;
    __syncthreads();
  }
  return prefix;
}

// Adds `key` (0 = not participating) to the histogram of pass `pass`.
__device__ __forceinline__ void hist_add(SelectSmem &sm, uint32_t key, int shift, uint32_t prefix,
                                         int pass) {
  if (key == 0) return;
  if (pass > 0 && (key >> (shift + 8)) != (prefix >> (shift + 8))) return;
  atomicAdd(&sm.hist[(key >> shift) & 255u], 1u);
}

// Bitonic sort of P (power of two) packed candidates in LDS, descending.
template <int NT>
__device__ void block_sort_desc(unsigned long long *a, int P) {
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P / 2; i += NT) {
        const int lo = 2 * stride * (i / stride) + (i % stride);
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const unsigned long long x = a[lo], y = a[hi];
        if ((x < y) == desc) { a[lo] = y; a[hi] = x; }
      }
      __syncthreads();
    }
  }
}

// Bitonic sort of P2 (a power of two, at most NT * E) packed candidates held
// in registers, E per thread at indices tid + NT * e, descending.  Partners
// closer than 64 are exchanged by lane shuffles, partners in other waves
// through LDS (two barriers), partners NT or more apart within the thread.
// `a` holds the input on entry (written before a barrier) and the result on
// return (after a barrier).
template <int NT, int E>
__device__ void bitonic_reg(unsigned long long *a, int P2) {
  const int tid = threadIdx.x;
  unsigned long long x[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + NT * e;
    x[e] = i < P2 ? a[i] : 0ull;
  }
  for (int size = 2; size <= P2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= NT) {
        // es = stride / NT, a power of two below E: one unrolled case each so
        // that every register index is a constant
#pragma unroll
        for (int es = 1; es < E; es <<= 1) {
          if (stride != NT * es) continue;
#pragma unroll
          for (int e = 0; e < E; ++e) {
            if (e & es) continue;
            const int i = tid + NT * e;
            const bool desc = (i & size) == 0;
            const unsigned long long lo = x[e], hi = x[e | es];
            if ((lo < hi) == desc) { x[e] = hi; x[e | es] = lo; }
          }
        }
      } else if (stride >= 64) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int i = tid + NT * e;
          if (i < P2) a[i] = x[e];
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int i = tid + NT * e;
          if (i < P2) {
            const unsigned long long y = a[i ^ stride];
            const bool keep_max = ((i & stride) == 0) == ((i & size) == 0);
            x[e] = keep_max ? (y > x[e] ? y : x[e]) : (y < x[e] ? y : x[e]);
          }
        }
        __syncthreads();
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int i = tid + NT * e;
          const unsigned long long y = __shfl_xor(x[e], stride);
          const bool keep_max = ((i & stride) == 0) == ((i & size) == 0);
          x[e] = keep_max ? (y > x[e] ? y : x[e]) : (y < x[e] ? y : x[e]);
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + NT * e;
    if (i < P2) a[i] = x[e];
  }
  __syncthreads();
}

// Bitonic sort of P2 packed candidates (a power of two, 64 < P2 <= NT) by
// the first P2 threads, one each; the other waves only take the barriers.
// Partners in other waves meet in LDS, alternately in `a` and `b` (P2
// entries each), so each such step needs one barrier.  The result is in `a`
// after a barrier.
template <int NT>
__device__ void bitonic_small(unsigned long long *a, unsigned long long *b, int P2) {
  const int tid = threadIdx.x;
  const bool act = tid < P2;   // whole waves: P2 is a multiple of 64
  unsigned long long x = act ? a[tid] : 0ull;
  int flip = 0;
  for (int size = 2; size <= P2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const bool keep_max = ((tid & stride) == 0) == ((tid & size) == 0);
      if (stride >= 64) {
        unsigned long long *buf = flip ? b : a;
        flip ^= 1;
        if (act) buf[tid] = x;
        __syncthreads();
        if (act) {
          const unsigned long long y = buf[tid ^ stride];
          x = keep_max ? (y > x ? y : x) : (y < x ? y : x);
        }
      } else if (act) {
        const unsigned long long y = __shfl_xor(x, stride);
        x = keep_max ? (y > x ? y : x) : (y < x ? y : x);
      }
    }
  }
  __syncthreads();   // every read of the last exchange buffer is done
  if (act) a[tid] = x;
  __syncthreads();
}

// Sorts the first n packed candidates of `a` descending (n <= kSortCap).
// `b`, when given, is a second buffer of kSortCap entries for the exchanges
// of n <= NT candidates.
template <int NT>
__device__ void sort_packed(unsigned long long *a, int n, unsigned long long *b = nullptr) {
  int P2 = 1;
  while (P2 < n) P2 <<= 1;
  for (int i = n + threadIdx.x; i < P2; i += NT) a[i] = 0ull;
  __syncthreads();
  if (P2 <= 64) {
    if (threadIdx.x < 64) {
      const int lane = lane_id();
      unsigned long long x = lane < P2 ? a[lane] : 0ull;
      x = wave_sort_desc64(x);
      if (lane < P2) a[lane] = x;
    }
    __syncthreads();
  } else if (b && P2 <= NT) {
    bitonic_small<NT>(a, b, P2);
  } else {
    static_assert(kSortCap % NT == 0, "sort_packed: kSortCap must be a multiple of NT");
    bitonic_reg<NT, kSortCap / NT>(a, P2);
  }
}

// Sorts the first n (<= kSortCap) packed candidates of `a` descending, all
// distinct, every key in [lo, hi]: a counting sort over kBinSortBins bins
// that split [lo, hi] evenly (a bin index monotone in the key), then each
// candidate's rank inside its bin by comparison with the bin's others.
// Six barriers, against about sixty for the bitonic network.  A bin with more
// than kBinSortMax candidates (values clustered or equal) sends the whole
// list to sort_packed instead.  `cnt` holds kBinSortBins + 32 words and `tmp`
// kSortCap entries of LDS, apart from `a`.
constexpr int kBinSortBins = 4096;
constexpr int kBinSortMax = 32;
template <int NT>
__device__ void sort_binned(unsigned long long *a, int n, uint32_t lo, uint32_t hi, uint32_t *cnt,
                            unsigned long long *tmp) {
  constexpr int NB = kBinSortBins, E = kSortCap / NT, PT = NB / NT;
  static_assert(kSortCap % NT == 0 && NB % NT == 0 && PT == 4, "sort_binned: layout");
  const int tid = threadIdx.x, lane = tid & 63;
  if (n <= 64) {
    sort_packed<NT>(a, n);
    return;
  }
  uint32_t *wsum = cnt + NB;      // NT / 64 words
  uint32_t *crowd = cnt + NB + 16;
  for (int i = tid; i < NB; i += NT) cnt[i] = 0u;
  if (tid == 0) *crowd = 0u;
  __syncthreads();
  // bin (descending: bin 0 holds the largest keys) and place in it; the
  // binary32 product rounds monotonically, so the bin never decreases with
  // the key
  const float scale = (float)NB / ((float)(hi - lo) + 1.0f);
  unsigned long long x[E];
  int bn[E], sl[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + NT * e;
    x[e] = 0ull;
    bn[e] = 0;
    sl[e] = 0;
    if (i < n) {
      x[e] = a[i];
      const uint32_t key = cand_key(x[e]);
      const int up = min(NB - 1, (int)((float)(key > lo ? key - lo : 0u) * scale));
      bn[e] = NB - 1 - up;
      sl[e] = (int)atomicAdd(&cnt[bn[e]], 1u);
    }
  }
  __syncthreads();
  // bin starts: exclusive prefix sum in place, PT bins per thread
  {
    const uint4 c = reinterpret_cast<const uint4 *>(cnt)[tid];
    const uint32_t s = c.x + c.y + c.z + c.w;
    const uint32_t mx = max(max(c.x, c.y), max(c.z, c.w));
    const uint32_t ex = block_scan_incl<NT>(s, wsum) - s;   // one barrier inside
    reinterpret_cast<uint4 *>(cnt)[tid] = make_uint4(ex, ex + c.x, ex + c.x + c.y, ex + c.x + c.y + c.z);
    if (__ballot(mx > (uint32_t)kBinSortMax) && lane == 0) *crowd = 1u;
  }
  __syncthreads();
  if (*crowd) {   // uniform: every thread reads the flag after the barrier
    sort_packed<NT>(a, n, tmp);
    return;
  }
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (tid + NT * e < n) tmp[cnt[bn[e]] + sl[e]] = x[e];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (tid + NT * e < n) {
      const int s = (int)cnt[bn[e]];
      const int t = bn[e] + 1 < NB ? (int)cnt[bn[e] + 1] : n;
      int rank = 0;
      for (int j = s; j < t; ++j) rank += tmp[j] > x[e] ? 1 : 0;
      a[s + rank] = x[e];
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- histories

// A row's history: n ids, the j-th (0 <= j < n) at p[hist_pos(h, j)].  Two
// layouts: the packed lists of hist_off (row r: hist_ids[off[r], off[r+1]),
// cap 0), and the rings of a decode state (row r: hist_ids[r * cap, ...), of
// which the last min(len[r], cap) appended ids count, the oldest at
// (len - n) mod cap).
struct HistRow {
  const int32_t *p;
  int64_t start, n, cap;
};

__device__ __forceinline__ HistRow hist_row(const LaunchArgs &a, int row) {
  HistRow h{a.hist_ids, 0, 0, 0};
  if (a.hist_cap > 0) {
    // (the scalar cache, invalidated when a kernel starts: a decode step
    // reads the row's length here and its own workgroup writes it at the end)
    int64_t len = load_scalar(a.hist_len + row);
    if (len < 0) len = 0;
    h.p = a.hist_ids + (int64_t)row * a.hist_cap;
    h.n = len < a.hist_cap ? len : a.hist_cap;
    h.start = (len - h.n) % a.hist_cap;
    h.cap = a.hist_cap;
  } else if (a.hist_off) {
    // (through the scalar cache: the offsets are not written while a kernel
    // runs, and the vector reads are not held up by them)
    const int64_t h0 = load_scalar(a.hist_off + row);
    h.p = a.hist_ids + h0;
    h.n = load_scalar(a.hist_off + row + 1) - h0;
  }
  return h;
}

__device__ __forceinline__ int64_t hist_pos(const HistRow &h, int64_t j) {
  const int64_t i = h.start + j;
  return (h.cap > 0 && i >= h.cap) ? i - h.cap : i;
}

// Writes a row's token.  In a decode step (src/engine.ts:1626-1644) the
// token's bookkeeping follows in the same lane: a row already done reports
// -1 and keeps its state; a stop id ends the row without joining the history
// (the stop check comes first, :1628); any other id joins the ring
// (tokenHistory.push, :1638).  A row the sampler leaves unresolved (-1)
// keeps its state.  The reads are issued together, before any write; the
// ring slot written is the oldest one, which no later read of this call
// needs (every read of the row's history precedes its token).
__device__ __forceinline__ void put_token(const LaunchArgs &a, int row, int token) {
  if (!a.dec_ring) {
    a.tokens[row] = token;
    return;
  }
  const int done = a.dec_done[row];
  int64_t len = a.dec_len[row];
  bool stop = false;
  for (int i = 0; i < a.dec_nstop; ++i) stop |= a.dec_stop[i] == token;
  if (done != 0 || token < 0) {
    a.tokens[row] = -1;
    return;
  }
  a.tokens[row] = token;
  if (stop) {
    a.dec_done[row] = 1;
    return;
  }
  if (len < 0) len = 0;
  a.dec_ring[(int64_t)row * a.hist_cap + len % a.hist_cap] = token;
  a.dec_len[row] = len + 1;
}

// ---------------------------------------------------------------- penalties

// src/sampler.ts:29-30 (v < 0 ? v * p : v / p, stored binary32) followed by
// the presence / frequency extension (v - freq * n) - pres, stored binary32.
__device__ __forceinline__ float penalise(float v, bool rep, uint32_t count, const RowPlan &P) {
  double x = (double)v;
  if (rep) x = (double)(float)(v < 0.0f ? x * P.rep : x / P.rep);
  if ((P.pen & kPenPF) && count > 0) {
    x = x - P.freq * (double)count;
    x = x - P.pres;
  }
  return (float)x;
}

// Penalty pre-pass for rows with presence / frequency penalties (and, on
// the large-k path, any penalty): one workgroup per row of pf_list.  The
// row's full history is counted into an LDS hash table of distinct ids (open
// addressing; the count word's top bit marks the ids of the last 128 entries),
// then every distinct id's logit is rewritten in place once.  A row whose
// distinct ids do not fit the table (kPenSlots, at most kPenProbe probes per
// insert) is counted instead by id ranges of kPenRange ids, one range at a
// time.  Logits are read and written only where penalised.
__device__ __forceinline__ uint32_t pen_hash(int id) {
  return ((uint32_t)id * 2654435761u) >> (32 - kPenBits);
}

// One row's penalties in place, by the whole workgroup of NT threads: `pdyn`
// holds pen_smem_bytes() of LDS, `full` is a shared flag.  The row's stores
// are issued when it returns; the caller orders them before any later read.
// on_write(id, value) sees every logit written.
struct PenNoHook {
  __device__ __forceinline__ void operator()(int, float) const {}
};
// The history entries pen_row counts start here: the repetition-only entries
// (before the last 128 without presence / frequency) are not counted, their
// count is not used.
__device__ __forceinline__ int64_t pen_start(const HistRow &h, const RowPlan &P) {
  const int64_t hl = h.n;
  const int64_t rep0 = (P.pen & kPenRep) ? hl - (hl < 128 ? hl : 128) : hl;   // history.slice(-128)
  return (P.pen & kPenPF) ? 0 : rep0;
}

// Thread tid's four history ids of the batch at t0 (-1 past the history).
template <int NT>
__device__ __forceinline__ void pen_request(const HistRow &h, int64_t t0, int (&ids)[4]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t t = t0 + tid + NT * c;
    ids[c] = t < h.n ? h.p[hist_pos(h, t)] : -1;
  }
}

// The table's penalised logits rewritten in place (every read of a thread's
// slots before any of its writes: no write can alias a later read, the slots
// hold distinct ids; every value before any store: a wait for a read issued
// before a store also waits for that store, so the stores go out back to
// back).
template <int NT, typename OnWrite = PenNoHook>
__device__ __forceinline__ void pen_apply(const uint32_t *pdyn, const RowPlan &P, float *rowp,
                                          OnWrite on_write = {}) {
  const int32_t *keys = reinterpret_cast<const int32_t *>(pdyn);
  const uint32_t *cnts = pdyn + kPenSlots;
  const int tid = threadIdx.x;
  const bool pf = (P.pen & kPenPF) != 0;
  constexpr int SPT = kPenSlots / NT;
  static_assert(kPenSlots % NT == 0, "pen_apply: slots per thread");
  int sid[SPT];
  float raw[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    sid[i] = keys[tid + NT * i];
    raw[i] = sid[i] >= 0 ? rowp[sid[i]] : 0.f;
  }
  float pv[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const uint32_t c = sid[i] >= 0 ? cnts[tid + NT * i] : 0u;
    pv[i] = penalise(raw[i], (c >> 31) != 0, pf ? (c & 0x7FFFFFFFu) : 0u, P);
    if (sid[i] >= 0) on_write(sid[i], pv[i]);
  }
#pragma unroll
  for (int i = 0; i < SPT; ++i)
    if (sid[i] >= 0) rowp[sid[i]] = pv[i];
}

struct PenNoSlot {
  __device__ __forceinline__ void operator()(int, uint32_t) const {}
};

// With `pre`, the caller has requested the first batch of ids (pen_request
// at pen_start) before reads of its own, whose waits then do not hold up the
// table.  With DEFER, a row whose distinct ids fit the table is not
// rewritten: on_slot(id, count word) sees each distinct id (count | rep bit
// 31), the table stays in pdyn, and the result is true; the caller applies
// the penalties (pen_apply, or from what on_slot kept).  Otherwise the row is
// rewritten in place and the result is false.
template <int NT, bool DEFER = false, typename OnWrite = PenNoHook, typename OnSlot = PenNoSlot>
__device__ __forceinline__ bool pen_row(const HistRow h, const RowPlan P, float *rowp, int V,
                                        uint32_t *pdyn, int32_t &full, OnWrite on_write = {},
                                        int (*pre)[4] = nullptr, OnSlot on_slot = {}) {
  int32_t *keys = reinterpret_cast<int32_t *>(pdyn);   // kPenSlots ids (-1: empty)
  uint32_t *cnts = pdyn + kPenSlots;                    // kPenSlots counts | rep bit
  const int tid = threadIdx.x;
  const int64_t hl = h.n;
  const int64_t rep0 = (P.pen & kPenRep) ? hl - (hl < 128 ? hl : 128) : hl;   // history.slice(-128)
  const bool pf = (P.pen & kPenPF) != 0;
  // Four ids per thread are requested before any is inserted, the first four
  // before the table is cleared.
  const int64_t tstart = pen_start(h, P);
  int ids[4];
  auto request = [&](int64_t t0) { pen_request<NT>(h, t0, ids); };
  if (pre) {
#pragma unroll
    for (int c = 0; c < 4; ++c) ids[c] = (*pre)[c];
  } else {
    request(tstart);
  }
  for (int i = tid; i < kPenSlots; i += NT) { keys[i] = -1; cnts[i] = 0; }
  if (tid == 0) full = 0;
  __syncthreads();
  bool over = false;
  auto insert = [&](int64_t t0) {
#pragma unroll 1
    for (int c = 0; c < 4; ++c) {
      const int64_t t = t0 + tid + NT * c;
      const int id = c == 0 ? ids[0] : c == 1 ? ids[1] : c == 2 ? ids[2] : ids[3];
      if (over || id < 0 || id >= V) continue;
      uint32_t hs = pen_hash(id);
      int probe = 0;
      for (; probe < kPenProbe; ++probe) {
        const int old = atomicCAS(&keys[hs], -1, id);
        if (old == -1 || old == id) break;
        hs = (hs + 1) & (kPenSlots - 1);
      }
      if (probe == kPenProbe) {
        over = true;
        continue;
      }
      atomicAdd(&cnts[hs], 1u);
      if (t >= rep0) atomicOr(&cnts[hs], 0x80000000u);
    }
  };
  // the first batch outside the loop: its wait counts the caller's later
  // reads exactly (a batch requested inside a loop is waited for with every
  // read before it)
  insert(tstart);
  for (int64_t t0 = tstart + 4 * NT; t0 < hl && !over; t0 += 4 * NT) {
    request(t0);
    insert(t0);
  }
  if (over) full = 1;
  __syncthreads();
  if (!full) {
    if (DEFER) {
      for (int i = tid; i < kPenSlots; i += NT)
        if (keys[i] >= 0) on_slot(keys[i], cnts[i]);
      return true;
    }
    pen_apply<NT>(pdyn, P, rowp, on_write);
    return false;
  }
  // too many distinct ids: count by id ranges (the table's LDS reused)
  uint32_t *counts = pdyn;                  // kPenRange
  uint32_t *repbits = pdyn + kPenRange;     // kPenRange / 32
  for (int lo = 0; lo < V; lo += kPenRange) {
    const int hi = min(lo + kPenRange, V);
    __syncthreads();
    for (int i = tid; i < kPenRange; i += NT) counts[i] = 0;
    for (int i = tid; i < kPenRange / 32; i += NT) repbits[i] = 0;
    __syncthreads();
    for (int64_t t = pf ? tid : rep0 + tid; t < hl; t += NT) {
      const int id = h.p[hist_pos(h, t)];
      if (id < lo || id >= hi) continue;
      atomicAdd(&counts[id - lo], 1u);
      if (t >= rep0) atomicOr(&repbits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    __syncthreads();
    for (int o = tid; o < hi - lo; o += NT) {
      const uint32_t n = counts[o];
      const bool rep = (repbits[o >> 5] >> (o & 31)) & 1u;
      if (n) {
        const float pv = penalise(rowp[lo + o], rep, pf ? n : 0u, P);
        rowp[lo + o] = pv;
        on_write(lo + o, pv);
      }
    }
  }
  return false;
}

__global__ __launch_bounds__(kPenThreads) void pen_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ uint32_t pdyn[];
  __shared__ int32_t full;
  const int row = ws.pf_list[blockIdx.x];
  pen_row<kPenThreads>(hist_row(a, row), ws.plans[row], a.logits + (int64_t)row * a.stride,
                       a.vocab, pdyn, full);
}

size_t pen_smem_bytes() {
  const size_t table = (size_t)kPenSlots * 8;
  const size_t ranges = (size_t)(kPenRange + kPenRange / 32) * 4;
  return table > ranges ? table : ranges;
}

// ---------------------------------------------------------------- replay

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x);

// k <= 64 slots of the scan in the lanes of one wave, sorted by (value, slot
// index): lane j holds c = (key << 32) | slot (key: f2key, -0 == +0; an
// empty slot, -Infinity, is 0) and the index rid of its logit (lanes >= k: c
// = ~0), and lane 0 holds the reference's minimum (the smallest slot among
// equal minima), key mk in slot mi.  A logit enters iff its key kL is above
// mk (NaN and -Infinity have key 0 and never do) and takes slot mi, c' =
// (kL, mi): lane 0 leaves, and lane j then holds the j-th smallest of lanes
// 1..k-1 and c', which is min(c[j + 1], max(c[j], c')).  For a logit that
// does not enter (kL <= mk, so c' <= c[0]) the same steps leave every lane
// as it is, so take_min needs no test: three lane-parallel steps (a wave
// shift by DPP, two 64-bit compares) and no scalar decision, which would
// wait for the vector unit at every logit.
__device__ __forceinline__ uint32_t wave_shl1_u32(uint32_t x) {   // lane j <- lane j + 1; lane 63 <- ~0
  return (uint32_t)__builtin_amdgcn_update_dpp((int)0xFFFFFFFF, (int)x, 0x130, 0xF, 0xF, false);
}

struct LaneSlots {
  unsigned long long c;
  int32_t rid;
  uint32_t mk;
  int mi, k;
  __device__ __forceinline__ explicit LaneSlots(int k_) : rid(-1), mk(0), mi(0), k(k_) {
    const int lane = lane_id();
    c = lane < k ? (unsigned long long)lane : ~0ull;
  }
  __device__ __forceinline__ void take_min(uint32_t kL, int idx) {
    const unsigned long long cL = ((unsigned long long)kL << 32) | (uint32_t)mi;
    const unsigned long long nx =
        ((unsigned long long)wave_shl1_u32((uint32_t)(c >> 32)) << 32) | wave_shl1_u32((uint32_t)c);
    const int32_t nr = (int32_t)wave_shl1_u32((uint32_t)rid);
    const bool below = c < cL;   // this lane's slot sorts below the new one
    const bool shift = nx < cL;  // so does the next lane's: this lane takes it
    const unsigned long long m = below ? cL : c;
    const int32_t mr = below ? idx : rid;
    c = shift ? nx : m;
    rid = shift ? nr : mr;
    mk = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(c >> 32));
    mi = __builtin_amdgcn_readfirstlane((int)(uint32_t)c);
  }
  // the logits of one 64-logit group (lane = logit) whose keys kx are above
  // the minimum at the group's start, in index order (those that no longer
  // are when their turn comes leave the slots as they are)
  __device__ __forceinline__ void scan64(uint32_t kx, int base) {
    unsigned long long cm = __ballot(kx > mk);
    while (cm) {
      const int L = (int)__ffsll((long long)cm) - 1;
      cm &= cm - 1;
      take_min(readlane_u32(kx, L), base + L);
    }
  }
  __device__ __forceinline__ void store(float *sv, int32_t *sid) const {
    if (lane_id() < k) {
      const int rs = (int)(uint32_t)c;
      sv[rs] = rid >= 0 ? key2f((uint32_t)(c >> 32)) : -INFINITY;
      sid[rs] = rid;
    }
  }
};

// LaneSlots for rows of fewer than 2^20 - 1 logits, one 64-bit word per
// lane: c = ~((key << 32) | (slot << 20) | index), the index field all ones
// for an empty slot, complemented so that lane 63, which a DPP shift leaves
// without a source, reads 0: a slot above every other.  Per logit: a wave
// shift of two dwords, two 64-bit compares, four selects, no index to move.
__device__ __forceinline__ uint32_t wave_shl1_zero(uint32_t x) {   // lane j <- lane j + 1; lane 63 <- 0
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x130, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t wave_shr1_u32(uint32_t x) {   // lane j <- lane j - 1; lane 0 <- 0
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x138, 0xF, 0xF, true);
}

struct PackedSlots {
  static constexpr uint32_t kNoIndex = 0xFFFFFu;
  unsigned long long c;
  // lane 0's low word with the index bits set, ~(mi << 20): the low word of
  // every compare key, and (xor the index) of the word a logit enters with
  uint32_t klo;
  int k;
  __device__ __forceinline__ explicit PackedSlots(int k_) : klo(0xFFFFFFFFu), k(k_) {
    const int lane = lane_id();
    c = lane < k ? ~(((unsigned long long)lane << 20) | kNoIndex) : 0ull;
  }
  __device__ __forceinline__ uint32_t min_key() const {   // mk
    return ~(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(c >> 32));
  }
  __device__ __forceinline__ void take_min(uint32_t kL, int idx) {
    // compared without its index (no slot sorts between (kL, mi) and the
    // new word, and a logit equal to the minimum must leave lane 0 as it is)
    const unsigned long long hi = (unsigned long long)~kL << 32;
    const unsigned long long cK = hi | klo;
    const unsigned long long cL = hi | (klo ^ (uint32_t)idx);
    const unsigned long long nx =
        ((unsigned long long)wave_shl1_zero((uint32_t)(c >> 32)) << 32) | wave_shl1_zero((uint32_t)c);
    const bool below = c > cK;   // complemented: this lane's slot sorts below the new one
    const bool shift = nx > cK;  // so does the next lane's: this lane takes it
    const unsigned long long m = below ? cL : c;
    c = shift ? nx : m;
    klo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)c) | kNoIndex;
  }
  __device__ __forceinline__ void scan64(uint32_t kx, int base) {
    unsigned long long cm = __ballot(kx > min_key());
    while (cm) {
      const int L = (int)__ffsll((long long)cm) - 1;
      cm &= cm - 1;
      take_min(readlane_u32(kx, L), base + L);
    }
  }
  // the keys of a row's first nblk blocks of 64 logits, from LDS (keys[64 b
  // + lane], 0 past the row), in index order.  When the row's first k
  // logits all have keys (the usual case) they fill slots 0..k-1 in order,
  // so the lanes are those k words sorted (one wave sort) rather than k
  // steps of take_min.
  __device__ __forceinline__ void scan_keys(const uint32_t *keys, int nblk) {
    if (nblk <= 0) return;
    const int lane = lane_id();
    uint32_t x = keys[lane];
    int from = 0;   // lanes of the first block still to scan
    const unsigned long long first = k >= 64 ? ~0ull : (1ull << k) - 1;
    if ((__ballot(lane < k && x != 0u) & first) == first) {
      c = lane < k ? ~(((unsigned long long)x << 32) | ((uint32_t)lane << 20) | (uint32_t)lane)
                   : 0ull;
      c = wave_sort_desc64(c);   // complemented: lane 0 the smallest (key, slot)
      klo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)c) | kNoIndex;
      from = k;
    }
    for (int b = 0; b < nblk; ++b) {
      const uint32_t xb = x;
      if (b + 1 < nblk) x = keys[(b + 1) * 64 + lane];   // the next block's read ahead of the scan
      scan64(b > 0 || lane >= from ? xb : 0u, b * 64);
    }
  }
  __device__ __forceinline__ void store(float *sv, int32_t *sid) const {
    if (lane_id() < k) {
      const unsigned long long v = ~c;
      const int rs = (int)((v >> 20) & 63u);
      const uint32_t ix = (uint32_t)v & kNoIndex;
      sv[rs] = ix != kNoIndex ? key2f((uint32_t)(v >> 32)) : -INFINITY;
      sid[rs] = ix != kNoIndex ? (int32_t)ix : -1;
    }
  }
  // The slots in the stable sort's order (src/sampler.ts:72-74: value
  // descending, equal values by slot ascending, empty slots last): lane j
  // (ascending by (key, slot)) goes to position (k - 1 - the last lane of its
  // key's run) + (j - the run's first lane).  sv / sid are indexed by that
  // position; sid holds the logit index.
  __device__ __forceinline__ void store_ordered(float *sv, int32_t *sid) const {
    const int lane = lane_id();
    const unsigned long long v = ~c;
    const uint32_t key = (uint32_t)(v >> 32);
    const uint32_t prev = wave_shr1_u32(key);
    const unsigned long long runs = __ballot(lane < k && (lane == 0 || key != prev));
    const unsigned long long upto = lane >= 63 ? ~0ull : (2ull << lane) - 1;
    const int first = 63 - __clzll(runs & upto);
    const unsigned long long above = runs & ~upto;
    const int last = above ? __ffsll((long long)above) - 2 : k - 1;
    if (lane < k) {
      const int pos = (k - 1 - last) + (lane - first);
      const uint32_t ix = (uint32_t)v & kNoIndex;
      sv[pos] = ix != kNoIndex ? key2f(key) : -INFINITY;
      sid[pos] = ix != kNoIndex ? (int32_t)ix : -1;
    }
  }
};
static_assert(kRowMaxVocab < (int)PackedSlots::kNoIndex, "PackedSlots: indices below the empty mark");

// Exact replace-min scan of src/sampler.ts:50-69 over the whole (penalised)
// row by one wave: slot j holds (sv[j], sid[j]); a logit enters iff it is
// strictly greater than the current minimum, into the first slot holding that
// minimum.  Logits are consumed in index order, 64 * BLK per step; the next
// step's loads are in flight while a step is scanned (one wave alone is
// bound by the latency of its reads).  BLK is what the caller's registers
// allow.
template <int BLK>
__device__ __forceinline__ void replay_row(const float *rowp, int vocab, int k, float *sv, int32_t *sid,
                                           const uint32_t *bkey = nullptr) {
  const int lane = lane_id();
  const bool in_regs = k <= 64;
  LaneSlots ls(k);
  auto scan64 = [&](uint32_t kx, int base) { ls.scan64(kx, base); };
  auto store_slots = [&]() { ls.store(sv, sid); };
  if (bkey && in_regs) {
    // bkey[b]: key of the largest logit of block b (64 logits).  A block
    // whose largest logit is not above the current minimum holds no logit
    // that enters, so it is not read.  Batches of up to BLK such blocks (in
    // index order, tested against the minimum when the batch is formed) are
    // read together, and the next batch's reads are issued before the
    // current batch is scanned: the scan of one batch hides the latency of
    // the next one's reads.
    const int nb = (vocab + 63) >> 6;
    int wb = -64;                      // window of 64 blocks being taken
    unsigned long long wm = 0;         // its blocks still to take
    auto form = [&](float (&x)[BLK], int (&blk)[BLK]) {
      int n = 0;
#pragma unroll
      for (int q = 0; q < BLK; ++q) {
        while (!wm && wb + 64 < nb) {
          wb += 64;
          const uint32_t kb = wb + lane < nb ? bkey[wb + lane] : 0u;
          wm = __ballot(kb > ls.mk);
        }
        blk[q] = -1;
        if (wm) {
          blk[q] = wb + (int)__ffsll((long long)wm) - 1;
          wm &= wm - 1;
          ++n;
        }
        const int e = blk[q] * 64 + lane;
        x[q] = rowp[blk[q] >= 0 && e < vocab ? e : 0];   // always a read inside the row
      }
      return n;
    };
    auto scan = [&](const float (&x)[BLK], const int (&blk)[BLK]) {
#pragma unroll
      for (int q = 0; q < BLK; ++q) {
        if (blk[q] >= 0) {
          const int e = blk[q] * 64 + lane;
          scan64(e < vocab ? f2key(x[q]) : 0u, blk[q] * 64);
        }
      }
    };
    float xa[BLK], xb[BLK];
    int ba[BLK], bb[BLK];
    int na = form(xa, ba);
    while (na > 0) {
      const int nb2 = form(xb, bb);
      scan(xa, ba);
      if (nb2 == 0) break;
      na = form(xa, ba);
      scan(xb, bb);
    }
    store_slots();
    return;
  }
  // the whole row, 64 * BLK logits per step; the reads of a step are only
  // issued when the step before is scanned (nothing uses them earlier);
  // `ok` marks the lanes inside the row
  float nx[BLK];
  uint32_t nok = 0;
#pragma unroll
  for (int q = 0; q < BLK; ++q) {
    const int e = q * 64 + lane;
    nx[q] = rowp[e < vocab ? e : 0];   // always a read inside the row
    nok |= (e < vocab ? 1u : 0u) << q;
  }
  if (in_regs) {
    for (int base = 0; base < vocab; base += 64 * BLK) {
      float x[BLK];
#pragma unroll
      for (int q = 0; q < BLK; ++q) x[q] = nx[q];
      const uint32_t ok = nok;
      if (base + 64 * BLK < vocab) {
        nok = 0;
#pragma unroll
        for (int q = 0; q < BLK; ++q) {
          const int e = base + 64 * BLK + q * 64 + lane;
          nx[q] = rowp[e < vocab ? e : 0];
          nok |= (e < vocab ? 1u : 0u) << q;
        }
      }
#pragma unroll
      for (int q = 0; q < BLK; ++q) scan64(((ok >> q) & 1u) ? f2key(x[q]) : 0u, base + q * 64);
    }
    store_slots();
    return;
  }
  // k > 64: the slots in LDS, the first minimum found by a wave search
  for (int j = lane; j < k; j += 64) { sv[j] = -INFINITY; sid[j] = -1; }
  float mv = -INFINITY;
  int mj = 0;
  for (int base = 0; base < vocab; base += 64 * BLK) {
    float x[BLK];
#pragma unroll
    for (int q = 0; q < BLK; ++q) x[q] = nx[q];
    const uint32_t ok = nok;
    if (base + 64 * BLK < vocab) {
      nok = 0;
#pragma unroll
      for (int q = 0; q < BLK; ++q) {
        const int e = base + 64 * BLK + q * 64 + lane;
        nx[q] = rowp[e < vocab ? e : 0];
        nok |= (e < vocab ? 1u : 0u) << q;
      }
    }
#pragma unroll
    for (int q = 0; q < BLK; ++q) {
      int done = -1;
      for (;;) {
        const unsigned long long b = __ballot(((ok >> q) & 1u) && x[q] > mv && lane > done);
        if (!b) break;
        const int L = __ffsll((long long)b) - 1;
        const float vL = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[q]), L));
        // a wave's LDS accesses complete in program order, so every lane's
        // rescan below observes this store
        if (lane == 0) { sv[mj] = vL; sid[mj] = base + q * 64 + L; }
        float bv = INFINITY;
        int bj = 0x7FFFFFFF;
        for (int j = lane; j < k; j += 64) {
          const float sj = sv[j];
          if (bj == 0x7FFFFFFF || sj < bv) { bv = sj; bj = j; }
        }
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) {
          const float ov = __shfl_xor(bv, m);
          const int oj = __shfl_xor(bj, m);
          const bool take = (oj != 0x7FFFFFFF) &&
                            (bj == 0x7FFFFFFF || ov < bv || (ov == bv && oj < bj));
          if (take) { bv = ov; bj = oj; }
        }
        mv = bv;
        mj = bj;
        done = L;
      }
    }
  }
}

// The staged replay's LDS beside the block keys: its list (a ring of
// kReplayRing words) and the keys of the row's first kHeadBlocks blocks,
// together in the fallback sort's kSortCap words.
constexpr int kReplayRing = 256;
constexpr int kHeadBlocks = 60;
static_assert(kReplayRing + 64 * kHeadBlocks <= 2 * kSortCap, "replay: ring and head in srt");

// Waves 1.. of the workgroup: keys[64 b + lane] = f2key of logit 64 b + lane
// (0 past the row) for the first h0 blocks, one block per wave at a time.
template <int NT>
__device__ __forceinline__ void replay_head_keys(const float *rowp, int V, int h0, uint32_t *keys) {
  constexpr int NW = NT / 64;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  if (wave == 0) return;
  constexpr int PER = (kHeadBlocks + NW - 2) / (NW - 1);
  float x[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = ((wave - 1) + (NW - 1) * q) * 64 + lane;
    x[q] = rowp[e < 64 * h0 && e < V ? e : 0];   // always a read inside the row
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int b = (wave - 1) + (NW - 1) * q, e = b * 64 + lane;
    if (b < h0) keys[e] = e < V ? f2key(x[q]) : 0u;
  }
}

// The slot replay of replay_row for k <= 64 with the whole workgroup, for
// the row kernel's rows whose draw needs it.  After logit i the slots hold
// the k largest logits of [0, i) (a logit enters iff it is above the
// smallest of them), so the k-th largest of the earlier blocks' largest
// logits is a lower bound of the scan's minimum at a block's start, and a
// block whose largest logit (bkey) is not above it holds no logit that
// enters.  Three kinds of work run at once, in steps separated by barriers:
//  - wave 1 keeps the k largest block keys sorted in its lanes (ascending,
//    updated as LaneSlots updates its slots) and lists, in index order, the
//    blocks whose key is above the smallest of them when they come (about
//    k + k ln(V / 64k) of the ceil(V / 64) blocks on random rows), a group
//    of G blocks ahead of the copies;
//  - waves 2.. copy the keys of the group listed before into LDS (two
//    alternating buffers);
//  - wave 0 scans the group copied before with PackedSlots::scan64 (the
//    steps of replay_row), reading LDS only.
// Every thread of the workgroup calls it with the same arguments; wave 0's
// ls holds the slots after the blocks below h0 (the dense head of the row,
// which its caller scans while the other waves take the block keys), and
// the list starts at block h0.  The slots end in sv / sid in the stable
// sort's order (PackedSlots::store_ordered).  bkey
// (nb = ceil(V / 64) words) lies at the start of `words` words of LDS, whose
// rest holds the buffers; ring (ring_cap words) holds the list, and pub (4
// words) the list's length and end, per step parity.  It returns false,
// having done nothing, when the buffers do not fit (the caller then runs
// replay_row).
constexpr int kStageBlocks = 32;   // G at most

template <int NT>
__device__ __forceinline__ bool replay_staged(const float *rowp, int V, int k, PackedSlots &ls,
                                              int h0, uint32_t *bkey, int words, uint32_t *ring,
                                              int ring_cap, int32_t *pub, float *sv,
                                              int32_t *sid) {
  constexpr int NW = NT / 64;
  static_assert(NW >= 3, "replay_staged: a scanning wave, a listing wave and copying waves");
  constexpr int PER = (kStageBlocks + NW - 3) / (NW - 2);   // blocks per copying wave and group
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int nb = (V + 63) >> 6;
  const int boff = (nb + 63) & ~63;
  const int G = min(kStageBlocks, (words - boff) / 128);
  if (G < 8 || ring_cap < 3 * G + 64 || V > kRowMaxVocab) return false;
  uint32_t *buf = bkey + boff;
  // wave 1's state
  uint32_t rk = lane < k ? 0u : 0xFFFFFFFFu;
  int w0 = 0, n = 0;
  int L = 0;   // blocks listed by the end of the previous step
  for (int t = 0;; ++t) {
    if (wave == 1) {
      while (n < (t + 1) * G && w0 < nb) {
        const uint32_t kb = w0 + lane < nb ? bkey[w0 + lane] : 0u;
        const uint32_t mk = (uint32_t)__builtin_amdgcn_readfirstlane((int)rk);
        unsigned long long cm = __ballot(kb > mk), ent = 0;
        while (cm) {
          const int Lb = (int)__ffsll((long long)cm) - 1;
          cm &= cm - 1;
          const uint32_t kL = readlane_u32(kb, Lb);
          ent |= (unsigned long long)(kL > rk) << Lb;   // lane 0's bits are the ones read
          rk = min(wave_shl1_u32(rk), max(rk, kL));
        }
        // the window's marked blocks, in index order, appended to the list
        // (blocks below h0 were scanned already)
        const unsigned long long em =
            (((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(ent >> 32))
              << 32) |
             (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ent)) &
            (w0 >= h0 ? ~0ull : w0 + 64 <= h0 ? 0ull : ~0ull << (h0 - w0));
        const int pos = n + (int)__builtin_amdgcn_mbcnt_hi(
                                (uint32_t)(em >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)em, 0u));
        if ((em >> lane) & 1ull) ring[pos % ring_cap] = (uint32_t)(w0 + lane);
        n += __popcll(em);
        w0 += 64;
      }
      if (lane == 0) {
        pub[2 * (t & 1)] = n;
        pub[2 * (t & 1) + 1] = w0 >= nb;
      }
    } else if (wave >= 2) {
      const int g = t - 1;   // listed by the end of the previous step
      if (g >= 0 && g * G < L) {
        const int j0 = g * G, nj = min(G, L - j0);
        uint32_t *dst = buf + (g & 1) * G * 64;
        float x[PER];
        int e[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) {
          const int j = (wave - 2) + (NW - 2) * q;
          e[q] = j < nj ? 64 * (int)ring[(j0 + j) % ring_cap] + lane : V;
          x[q] = rowp[e[q] < V ? e[q] : 0];   // always a read inside the row
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
          const int j = (wave - 2) + (NW - 2) * q;
          if (j < nj) dst[j * 64 + lane] = e[q] < V ? f2key(x[q]) : 0u;
        }
      }
    } else {
      const int g = t - 2;   // copied in the previous step
      if (g >= 0 && g * G < L) {
        const int j0 = g * G, nj = min(G, L - j0);
        const uint32_t *src = buf + (g & 1) * G * 64;
        const uint32_t bl = lane < nj ? ring[(j0 + lane) % ring_cap] : 0u;
        uint32_t xn = src[lane];
        for (int j = 0; j < nj; ++j) {
          const uint32_t x = xn;
          if (j + 1 < nj) xn = src[(j + 1) * 64 + lane];   // the next block's read ahead of the scan
          ls.scan64(x, 64 * (int)readlane_u32(bl, j));
        }
      }
    }
    __syncthreads();
    L = pub[2 * (t & 1)];
    const bool done = pub[2 * (t & 1) + 1] != 0;
    if (done && (t - 1) * G >= L) break;   // groups 0..t-2 scanned: every listed block
  }
  if (wave == 0) ls.store_ordered(sv, sid);
  return true;
}

// ---------------------------------------------------------------- row completion

struct TailSmem {
  int32_t n_sel, replay, cutoff, pick;
  int32_t m, f1, f2, hit;
  double sum;
  double wtot[16];
};

struct RowScratch {          // LDS arrays of at least k entries each
  uint32_t *skey;
  int32_t *sids;
  float *sprob;
  double *sp;
  float *rsv;
  int32_t *rsid;
};

// atomicMin(dst, i) for the first lane of the wave whose pred holds, i rising
// with the lane: one LDS atomic per wave instead of one per qualifying lane
// (they all hit one word and would be serialised).
__device__ __forceinline__ void first_min(bool pred, int i, int32_t *dst) {
  const unsigned long long b = __ballot(pred);
  if (b && lane_id() == __ffsll((long long)b) - 1) atomicMin(dst, i);
}

// Block-parallel tail of src/sampler.ts:79-117 over n >= 2 sorted candidate
// keys s.skey[0, n) (descending), by NT threads.  Leaves the probabilities in
// s.sprob and f.cutoff, f.pick.
//   sumProb is a block sum in tree order, not the reference's sequential
//   order: the difference is a few binary64 ulps, far inside the binary32
//   rounding of the probabilities.
//   cumProb and the draw's r are exact, as in wave_tail: over the prefix of
//   probabilities that are 0 or in [2^-29, 1] (the probabilities descend, so
//   the others form a suffix starting at m) every partial sum below 2 is
//   exact in any order, so cumProb is a block prefix sum there and the draw
//   is the first index whose prefix reaches u*keptSum.  Past m, one thread
//   continues the reference's sequential loops.
template <int NT>
__device__ __forceinline__ void tail_block(int n, const RowPlan &P, double u, RowScratch s, TailSmem &f) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NW = NT / 64;
  const double maxl = (double)key2f(s.skey[0]);
  const double inv_temp = 1.0 / P.temperature;
  double local = 0;
  for (int i = tid; i < n; i += NT) {
    const double p = exp(((double)key2f(s.skey[i]) - maxl) * inv_temp);
    s.sp[i] = p;
    local += p;
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) local += __shfl_xor(local, d);
  if (lane == 0) f.wtot[wave] = local;
  if (tid == 0) { f.m = n; f.f1 = n; f.f2 = n; f.hit = n; }
  __syncthreads();
  double sum = 0;
  for (int w = 0; w < NW; ++w) sum += f.wtot[w];
  for (int i = tid; i < n; i += NT) {
    const float prob = (float)((double)(float)s.sp[i] / sum);
    s.sprob[i] = prob;
    const double pd = (double)prob;
    first_min(!(pd == 0.0 || (pd >= 0x1p-29 && pd <= 1.0)), i, &f.m);
  }
  __syncthreads();
  const double thr = P.min_p * (double)s.sprob[0];
  for (int i = tid; i < n; i += NT) first_min(i > 0 && (double)s.sprob[i] < thr, i, &f.f1);
  const int m = f.m;
  // exact prefix sums over [0, m), into s.sp
  double carry = 0;
  bool exact = true;
  for (int base = 0; base < m; base += NT) {
    const int i = base + tid;
    double c = wave_scan_incl_f64(i < m ? (double)s.sprob[i] : 0.0);
    __syncthreads();   // the previous page's totals are read
    if (lane == 63) f.wtot[wave] = c;
    __syncthreads();
    double add = carry, tot = carry;
    for (int w = 0; w < NW; ++w) {
      if (w < wave) add += f.wtot[w];
      tot += f.wtot[w];
    }
    c += add;
    if (i < m) s.sp[i] = c;
    first_min(i < m && c >= P.top_p, i, &f.f2);
    carry = tot;
    exact = exact && tot < 2.0;
  }
  __syncthreads();
  if (!exact) {   // partial sums reached 2: the sequential loops from the start
    if (tid == 0) f.m = 0;
    __syncthreads();
  }
  const int mm = f.m;
  if (tid == 0) {
    int f1 = f.f1, f2 = f.f2 < mm ? f.f2 : n;
    int cut;
    if (f1 <= f2 && f1 <= mm) cut = f1;          // a min-p break at or before m
    else if (f2 < mm) cut = f2 + 1;              // a top-p break before m
    else {                                       // the reference's loop from m on
      double cum = mm > 0 ? s.sp[mm - 1] : 0.0;
      cut = n;
      for (int i = mm; i < n; ++i) {
        if (i > 0 && (double)s.sprob[i] < thr) { cut = i; break; }
        cum += (double)s.sprob[i];
        s.sp[i] = cum;
        if (cum >= P.top_p) { cut = i + 1; break; }
      }
    }
    f.cutoff = cut;
  }
  __syncthreads();
  const int cut = f.cutoff;
  const double kept = s.sp[cut - 1];   // keptSum equals cumProb at cutoff - 1
  const double r0 = u * kept;
  if (cut <= mm) {
    for (int i = tid; i < cut; i += NT) first_min(s.sp[i] >= r0, i, &f.hit);
    __syncthreads();
    if (tid == 0) f.pick = f.hit < cut ? f.hit : cut - 1;
  } else if (tid == 0) {
    double r = r0;
    int pick = cut - 1;
    for (int i = 0; i < cut; ++i) {
      r -= (double)s.sprob[i];
      if (r <= 0) { pick = i; break; }
    }
    f.pick = pick;
  }
  __syncthreads();
}

// Completes a top-k row.  `srt` holds n_sel packed candidates, every logit
// with key >= T (the exact k-th largest key; all candidates when fewer than
// k), sorted descending.  closed_form: no slot was ever evicted (at most k
// finite logits), so equal values are in index order as sorted.
// need_replay: the candidates are not trustworthy (a list overflowed).
// Writes the token and the optional outputs of `row`.
template <int NT>
__device__ __forceinline__ void finish_row(const LaunchArgs &a, const RowPlan &P, int row, const float *rowp,
                           unsigned long long *srt, int n_sel, uint32_t T, bool closed_form,
                           bool need_replay, RowScratch s, TailSmem &f) {
  const int tid = threadIdx.x;
  const int k = P.k;
  int n = 0;
  bool boundary_tie = false, internal_tie = false;
  if (!need_replay) {
    n = n_sel < k ? n_sel : k;
    boundary_tie = n_sel > k;
    int tie = 0;
    for (int i = tid; i < n; i += NT) {
      const uint32_t key = cand_key(srt[i]);
      s.skey[i] = key;
      s.sids[i] = (int32_t)cand_idx(srt[i]);
      if (i + 1 < n) tie |= key == cand_key(srt[i + 1]);
    }
    internal_tie = __syncthreads_or(tie) != 0;   // also completes skey, sids
    if (closed_form) { boundary_tie = false; internal_tie = false; }
    // the candidate outputs must carry the reference's exact order
    if ((boundary_tie || internal_tie) && a.want_cands) need_replay = true;
  }
  if (tid == 0) f.replay = 0;
  __syncthreads();

  // tail, src/sampler.ts:76-117; runs twice when a tie group holds the draw
  const double u = a.uniforms[row];
  for (int attempt = 0; attempt < 2; ++attempt) {
    if (need_replay) {
      if (tid < 64) replay_row<NT == kRowThreads ? 8 : 32>(rowp, a.vocab, k, s.rsv, s.rsid);
      __syncthreads();
      if (tid == 0) f.n_sel = 0;
      __syncthreads();
      for (int j = tid; j < k; j += NT) {
        if (s.rsid[j] >= 0) {
          const int p = atomicAdd(&f.n_sel, 1);
          srt[p] = pack_cand(f2key(s.rsv[j]), (uint32_t)j);   // ties by slot
        }
      }
      __syncthreads();
      n = f.n_sel;
      sort_packed<NT>(srt, n);
      for (int i = tid; i < n; i += NT) {
        s.skey[i] = cand_key(srt[i]);
        s.sids[i] = s.rsid[cand_idx(srt[i])];
      }
      if (tid == 0) f.replay = 1;
      __syncthreads();
      boundary_tie = internal_tie = false;
    }

    if (n >= 2) {
      tail_block<NT>(n, P, u, s, f);
    } else {
      if (tid == 0) { f.cutoff = n; f.pick = n == 1 ? 0 : -1; }
      __syncthreads();
    }

    if (attempt == 0 && !need_replay && (boundary_tie || internal_tie)) {
      // Order inside a group of equal values follows the slot history; it
      // changes the token only if the drawn position lies in such a group.
      const int pick = f.pick;
      bool hit = false;
      if (pick >= 0) {
        const uint32_t kp = s.skey[pick];
        hit = (pick > 0 && s.skey[pick - 1] == kp) || (pick + 1 < n && s.skey[pick + 1] == kp) ||
              (boundary_tie && kp == T);
      }
      if (hit) { need_replay = true; continue; }
    }
    break;
  }

  const int cs = a.cand_stride;
  if (tid == 0) {
    const int pick = f.pick;
    put_token(a, row, pick >= 0 ? s.sids[pick] : 0);
    if (a.cand_count_out) a.cand_count_out[row] = n;
    if (a.cutoff_out) a.cutoff_out[row] = f.cutoff;
    if (a.row_flags) {
      uint32_t fl = 0;
      if (f.replay) fl |= HS_ROW_REPLAYED;
      if (boundary_tie || internal_tie || f.replay) fl |= HS_ROW_TIES;
      if (n < 2) fl |= HS_ROW_SINGLE;
      a.row_flags[row] = fl;
    }
  }
  if (a.cand_ids || a.cand_probs) {
    for (int i = tid; i < n && i < cs; i += NT) {
      if (a.cand_ids) a.cand_ids[(int64_t)row * cs + i] = s.sids[i];
      if (a.cand_probs) a.cand_probs[(int64_t)row * cs + i] = n >= 2 ? s.sprob[i] : 1.0f;
    }
  }
}

// Writes the greedy result: first index of the maximum (src/sampler.ts:37-45);
// `best` is the packed maximum over the row (0 = no non-NaN logit).
// x0: the row's (penalised) logit 0.
__device__ __forceinline__ void write_greedy(const LaunchArgs &a, int row, float x0,
                             unsigned long long best) {
  int token = best ? (int)cand_idx(best) : 0;
  if (isnan(x0)) token = 0;   // bestVal = logits[0] = NaN: nothing is '>' it
  put_token(a, row, token);
  if (a.cand_count_out) a.cand_count_out[row] = 0;
  if (a.cutoff_out) a.cutoff_out[row] = 0;
  if (a.row_flags) a.row_flags[row] = HS_ROW_GREEDY;
}

struct SelResult {
  int n_sel;
  uint32_t T;
};

// Gathers the entries get(0 .. n_ent) with key >= lo into srt after selecting
// the exact k-th largest key T among them (all of them when fewer than k).
// Returns T and n_sel (entries with key >= T) sorted descending in srt, or
// n_sel = -1 when more than kSortCap entries lie at or above T.  (Not inlined:
// a rare path.  Its arguments and result travel in registers, so the callers
// need no scratch memory.)
template <int NT, typename GetEnt>
__device__ SelResult select_into(int n_ent, GetEnt get, uint32_t lo, int k,
                                 unsigned long long *srt, SelectSmem &sm, TailSmem &f) {
  const int tid = threadIdx.x;
  int total = 0;
  const uint32_t T = block_select_fast<NT>(
      k,
      [&](int shift, uint32_t prefix, int pass) {
        for (int p = tid; p < n_ent; p += NT) {
          const uint32_t key = cand_key(get(p));
          hist_add(sm, key >= lo ? key : 0u, shift, prefix, pass);
        }
      },
      sm, &total);
  const uint32_t X = T ? T : (lo ? lo : 1u);   // fewer than k: keep them all
  if (tid == 0) f.n_sel = 0;
  __syncthreads();
  for (int p = tid; p < n_ent; p += NT) {
    const unsigned long long c = get(p);
    if (cand_key(c) >= X) {
      const int q = atomicAdd(&f.n_sel, 1);
      if (q < kSortCap) srt[q] = c;
    }
  }
  __syncthreads();
  const int n_sel = f.n_sel;
  if (n_sel > kSortCap) return {-1, T};
  sort_packed<NT>(srt, n_sel);
  return {n_sel, T};
}

// ---------------------------------------------------------------- row kernel

// A row is read in rounds.  Round 0 holds kR0NV float4 per thread (24576
// logits); every later round kRowNV (32768 logits).  In a round whose first
// float4 is fb, thread t holds the float4s fb + t + j * kRowThreads, so every
// wave reads 1 KiB contiguous per load instruction and all waves finish a
// round together.  Round 0 is small so that the bound it fixes is ready
// early, while rounds 1 and 2 are both in flight.

__device__ __forceinline__ int round_base(int r) {
  return r == 0 ? 0 : kR0F4 + (r - 1) * kRoundF4;
}

__device__ __forceinline__ int row_rounds(int V) {
  const int nf4 = (V + 3) >> 2;
  return nf4 <= kR0F4 ? 1 : 1 + (nf4 - kR0F4 + kRoundF4 - 1) / kRoundF4;
}

__device__ __forceinline__ int slot_elem(int fb, int tid, int j) {
  return 4 * (fb + tid + j * kRowThreads);
}

__device__ __forceinline__ int uniform_i32(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Row reads go through buffer resources.  A read at or past a resource's
// num_records returns 0 and touches no memory, so no read of the row needs a
// branch around it, and the compiler counts the reads in flight exactly: a
// round is waited for only when it is used, never at a barrier or a branch.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kReadNT = 2;   // cache policy of a streamed read: nt

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}

// The last <= 128 ids of a row's history (src/sampler.ts:26,
// history.slice(-128)), the t-th to thread t, requested with one buffer load
// (threads past them read outside the resource: 0, no memory touched).
struct HistTail {
  int id;
  int n;
};

__device__ __forceinline__ HistTail hist_tail(const LaunchArgs &a, int row, int tid) {
  const HistRow h = hist_row(a, row);
  const int n = (int)(h.n < 128 ? h.n : 128);
  const int64_t j0 = h.n - n;
  const int32_t *p = h.p + j0;
  uint32_t bytes = 4u * (uint32_t)n, off = 4u * (uint32_t)tid;
  if (h.cap > 0) {   // a ring: the window may wrap
    p = h.p;
    bytes = 4u * (uint32_t)h.cap;
    off = tid < n ? 4u * (uint32_t)hist_pos(h, j0 + tid) : bytes;
  }
  HistTail t;
  t.id = (int)__builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p, bytes), off, 0, 0);
  t.n = n;
  return t;
}

// The row as the rounds read it.  With VEC (16-byte aligned rows) x4 covers
// the lim = 4 * floor(V / 4) logits of whole float4s, and the fewer than four
// past them (the tail) are read apart; without VEC the rounds read the row by
// element through x1 and lim = V.
struct RowSrc {
  rsrc_t x4, x1;
  int lim;
};

// One round into registers.  Slots past lim read as 0 here; clip_rd turns
// them into NaN (never a candidate) once the round has arrived.
template <int NV, bool VEC>
__device__ __forceinline__ void load_rd(float (&v)[NV][4], const RowSrc &src, int fb, int tid) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int f = fb + tid + j * kRowThreads;
    if (VEC) {
      const auto t = __builtin_amdgcn_raw_buffer_load_b128(src.x4, f * 16, 0, kReadNT);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[j][q] = __uint_as_float(t[q]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[j][q] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(src.x1, (4 * f + q) * 4, 0, kReadNT));
    }
  }
}

template <int NV>
__device__ __forceinline__ void clip_rd(float (&v)[NV][4], int fb, int tid, int lim) {
  if (4 * (fb + NV * kRowThreads) <= lim) return;   // uniform: only a round reaching past lim
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = slot_elem(fb, tid, j);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (e + q >= lim) v[j][q] = __builtin_nanf("");
  }
}

// Logits whose id is in the repetition set (bitmap) leave the stream: their
// penalised values join the selection separately.
template <int NV>
__device__ __forceinline__ void mask_penalised(float (&v)[NV][4], int fb, int tid, int V,
                                               const uint32_t *bitmap) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = slot_elem(fb, tid, j);
    if (e < V) {
      const uint32_t bits = (bitmap[e >> 5] >> (e & 31)) & 0xFu;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (bits & (1u << q)) v[j][q] = __builtin_nanf("");
    }
  }
}

// Appends every logit of the round at or above xf to the wave's own segment
// of the candidate list; cnt (wave-uniform) counts them, also past kSegCap,
// where they are no longer stored.  No LDS round trip: a position is the
// count so far plus the lanes below in the ballot.  Logits in the repetition
// set are appended with their raw values and dropped at the end of the row.
template <int NV>
__device__ __forceinline__ void append_rd(const float (&v)[NV][4], int fb, int tid, float xf,
                                          unsigned long long *seg, int &cnt) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    // one ballot per float4 first: most hold no candidate (NaN is ignored)
    const float m = fmaxf(fmaxf(v[j][0], v[j][1]), fmaxf(v[j][2], v[j][3]));
    if (!__ballot(m >= xf)) continue;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool pass = v[j][q] >= xf;
      const unsigned long long b = __ballot(pass);
      if (b) {
        const int p = cnt + (int)lanes_below(b);
        if (pass && p < kSegCap)
          seg[p] = pack_cand(f2key(v[j][q]), (uint32_t)(slot_elem(fb, tid, j) + q));
        cnt = uniform_i32(cnt + __popcll(b));
      }
    }
  }
}

// Packed maximum (value, then lowest index) of a round, folded into `best`.
template <int NV>
__device__ __forceinline__ unsigned long long greedy_rd(const float (&v)[NV][4], int fb, int tid,
                                                        unsigned long long best) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = slot_elem(fb, tid, j);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t key = f2key(v[j][q]);
      const unsigned long long c = key ? pack_cand(key, (uint32_t)(e + q)) : 0ull;
      best = c > best ? c : best;
    }
  }
  return best;
}

template <int NV>
__device__ __forceinline__ float rd_max(const float (&v)[NV][4]) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) m = fmaxf(m, v[j][q]);   // NaN is ignored
  return m;
}


// Maximum of one key per lane over the wave (DPP row shifts and row
// broadcasts, then lane 63), returned wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  // row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143
  uint32_t y;
  y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x111, 0xF, 0xF, false); x = x > y ? x : y;
  y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x112, 0xF, 0xF, false); x = x > y ? x : y;
  y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x114, 0xF, 0xF, false); x = x > y ? x : y;
  y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x118, 0xF, 0xF, false); x = x > y ? x : y;
  y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x142, 0xA, 0xF, false); x = x > y ? x : y;
  y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x143, 0xC, 0xF, false); x = x > y ? x : y;
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// The j-th largest of one key per lane (1 <= j <= 4, multiset order; 0 when
// fewer than j lanes hold a non-zero key): j rounds of wave maximum, each
// retiring one lane that holds it.
__device__ __forceinline__ uint32_t wave_jth_largest(uint32_t key, int j) {
  const int lane = lane_id();
  uint32_t m = 0;
  for (int t = 0; t < j; ++t) {
    m = wave_max_u32(key);
    const unsigned long long b = __ballot(key == m);
    if (lane == (int)__ffsll((long long)b) - 1) key = 0;
  }
  return m;
}

// Largest t in [lo, hi] with at least k of the keys >= t: a ballot binary
// search over the bits in which lo and hi differ (all others are shared).
template <int SLOTS>
__device__ __forceinline__ uint32_t wave_search(const uint32_t (&key)[SLOTS], int slots, int k,
                                                uint32_t lo, uint32_t hi) {
  const uint32_t diff = lo ^ hi;
  if (!diff) return lo;
  const int hb = 31 - __builtin_clz(diff);
  uint32_t t = hb == 31 ? 0u : (lo & ~((2u << hb) - 1u));
  for (int b = hb; b >= 0; --b) {
    const uint32_t c = t | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
      if (SLOTS <= 4 || s < slots) cnt += __popcll(__ballot(key[s] >= c));
    if (cnt >= k) t = c;
  }
  return t;
}

// Exact k-th largest of n keys list[0, n) (n <= kRowThreads) by one wave,
// given that at least k of them are >= lo.  0 when n < k.
__device__ __forceinline__ uint32_t wave_kth_of_list(const uint32_t *list, int n, int k,
                                                     uint32_t lo) {
  n = uniform_i32(n);
  lo = (uint32_t)uniform_i32((int)lo);
  if (n < k) return 0u;
  const int lane = lane_id();
  if (n <= 128) {
    uint32_t key[2];
    key[0] = lane < n ? list[lane] : 0u;
    key[1] = lane + 64 < n ? list[lane + 64] : 0u;
    const uint32_t hi = wave_max_u32(key[0] > key[1] ? key[0] : key[1]);
    return wave_search<2>(key, 2, k, lo, hi);
  }
  if (n <= 256) {
    uint32_t key[4], hi = 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      key[s] = lane + 64 * s < n ? list[lane + 64 * s] : 0u;
      hi = key[s] > hi ? key[s] : hi;
    }
    hi = wave_max_u32(hi);
    return wave_search<4>(key, 4, k, lo, hi);
  }
  const int slots = (n + 63) >> 6;
  uint32_t key[kRowWaves];
  uint32_t hi = 0;
#pragma unroll
  for (int s = 0; s < kRowWaves; ++s) {
    const int i = lane + 64 * s;
    key[s] = (s < slots && i < n) ? list[i] : 0u;
    hi = key[s] > hi ? key[s] : hi;
  }
  hi = wave_max_u32(hi);
  return wave_search<kRowWaves>(key, slots, k, lo, hi);
}

// Tightens the bound mid-row, by one wave: T = the exact k-th largest key of
// the n candidates cbuf[0, n) (k <= n <= 64 * SLOTS, all with a key >= lo),
// a lower bound of the row's k-th largest; the candidates below T are
// dropped in place.  Returns T and the number kept.
template <int SLOTS>
__device__ __forceinline__ uint32_t wave_refine(unsigned long long *cbuf, int n, int k, uint32_t lo,
                                                int *kept) {
  const int lane = lane_id();
  unsigned long long c[SLOTS];
  uint32_t key[SLOTS], hi = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int i = lane + 64 * s;
    c[s] = i < n ? cbuf[i] : 0ull;
    key[s] = cand_key(c[s]);
    hi = key[s] > hi ? key[s] : hi;
  }
  hi = wave_max_u32(hi);
  const uint32_t T = wave_search<SLOTS>(key, SLOTS, k, lo ? lo : 1u, hi);
  int m = 0;   // every read above precedes the writes below (one wave, LDS in order)
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const bool pass = key[s] >= T;
    const unsigned long long b = __ballot(pass);
    if (pass) cbuf[m + (int)lanes_below(b)] = c[s];
    m += __popcll(b);
  }
  *kept = m;
  return T;
}

// A bound from a snapshot of the candidate segments, by one wave while the
// other waves keep appending: the exact k-th largest key among the entries
// published so far (wcnt[w] of segment w, at most 32 each), leaving out the
// logits of the repetition set.  A wave writes its entries before it
// publishes their count and a wave's LDS accesses complete in order, so every
// entry below a published count is whole.  A result above lo has at least k
// such keys at or above it; lo is returned when the snapshot does not fit.
__device__ __forceinline__ uint32_t wave_snapshot_bound(const unsigned long long *cbuf,
                                                        const int32_t *wcnt, int k, uint32_t lo,
                                                        const uint32_t *bitmap, bool rep) {
  const int lane = lane_id();
  const int c = lane < kRowWaves ? __atomic_load_n(wcnt + lane, __ATOMIC_RELAXED) : 0;
  int tot = c, cmax = c;
#pragma unroll
  for (int m = 1; m < kRowWaves; m <<= 1) {
    tot += __shfl_xor(tot, m);
    const int o = __shfl_xor(cmax, m);
    cmax = o > cmax ? o : cmax;
  }
  tot = uniform_i32(tot);
  cmax = uniform_i32(cmax);
  if (cmax > 32 || tot < k) return lo;
  const int w = lane & (kRowWaves - 1);
  const int cw = __shfl(c, w);
  uint32_t key[8], hi = 0;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int q = (lane >> 4) + 4 * t;
    uint32_t kk = 0;
    if (q < cw) {
      const unsigned long long e = cbuf[w * kSegCap + q];
      const uint32_t id = cand_idx(e);
      kk = (rep && ((bitmap[id >> 5] >> (id & 31)) & 1u)) ? 0u : cand_key(e);
    }
    key[t] = kk;
    hi = kk > hi ? kk : hi;
  }
  hi = wave_max_u32(hi);
  if (hi <= lo) return lo;
  return wave_search<8>(key, 8, k, lo ? lo : 1u, hi);
}

// Sorted top-64 of n distinct packed candidates cbuf[0, n) (n <= kRowThreads)
// by ranking: G threads per candidate count the larger ones, the candidate of
// rank r < 64 lands in top[r]; the key of rank 64 goes to *key64 (0 if none).
// top[] must hold zeros beforehand.  Ends with a barrier.
__device__ __forceinline__ void rank_top64(const unsigned long long *cbuf, int n,
                                           unsigned long long *top, uint32_t *key64) {
  const int tid = threadIdx.x;
  int G = 1;
  while (G < 64 && 2 * G * n <= kRowThreads) G <<= 1;
  const int i = tid / G, g = tid & (G - 1);
  const unsigned long long x = i < n ? cbuf[i] : ~0ull;
  int rank = 0;
  if (i < n) {
    int j = g;
    for (; j + 3 * G < n; j += 4 * G) {
      const unsigned long long y0 = cbuf[j], y1 = cbuf[j + G], y2 = cbuf[j + 2 * G],
                               y3 = cbuf[j + 3 * G];
      rank += (int)(y0 > x) + (int)(y1 > x) + (int)(y2 > x) + (int)(y3 > x);
    }
    for (; j < n; j += G) rank += (int)(cbuf[j] > x);
  }
  for (int m = 1; m < G; m <<= 1) rank += __shfl_xor(rank, m);
  if (i < n && g == 0) {
    if (rank < 64) top[rank] = x;
    if (rank == 64) *key64 = cand_key(x);
  }
  __syncthreads();
}


// Tail of src/sampler.ts:76-117 for n <= 64 candidates held one per lane
// (value keys `key`, sorted descending), by one wave.
//   sumProb (src/sampler.ts:82-86) adds unrounded binary64 terms, so it runs
//   as a sequential chain in the reference's order: the terms go through `sp`
//   (64 doubles of LDS) and are read back by broadcast.
//   cumProb and the draw's r (src/sampler.ts:91-116) add and subtract the
//   binary32 probabilities.  When every probability is 0 or in [2^-29, 1],
//   each is a multiple of 2^-52, so every partial sum below 2 is exact in
//   binary64 in any order; then cumProb is a wave prefix sum, and r stays
//   exactly u*keptSum - cumProb until its sign flips (a rounded difference
//   keeps the sign of the exact one), so the draw is the first index whose
//   prefix reaches u*keptSum.  Otherwise the sums run as sequential chains
//   through `sp` with every lane stopping at its own index (later terms are
//   replaced by +0, which leaves a running sum unchanged).
// Returns the picked position (-1 when n == 0) and writes the cutoff and each
// lane's normalised probability.
__device__ __forceinline__ int wave_tail(uint32_t key, int n, const RowPlan &P, double u, int *cutoff,
                         float *prob_out, double *sp) {
  const int lane = lane_id();
  if (n < 2) {
    *cutoff = n;
    *prob_out = 1.0f;
    return n == 1 ? 0 : -1;
  }
  n = uniform_i32(n);
  const int n8 = (n + 7) & ~7;
  const double v = (double)key2f(key);
  const double maxl = readlane_f64(v, 0);
  const double inv_temp = 1.0 / P.temperature;
  const double p = lane < n ? exp((v - maxl) * inv_temp) : 0.0;
  sp[lane] = p;   // a wave's LDS accesses complete in order
  double sum = 0;
  for (int j = 0; j < n8; j += 8) {
#pragma unroll
    for (int q = 0; q < 8; ++q) sum += sp[j + q];
  }
  const float prob = (float)((double)(float)p / sum);
  *prob_out = prob;
  const double pd = lane < n ? (double)prob : 0.0;
  bool exact = !__ballot(lane < n && !(pd == 0.0 || (pd >= 0x1p-29 && pd <= 1.0)));
  double cum = 0;
  if (exact) {
    cum = wave_scan_incl_f64(pd);
    exact = readlane_f64(cum, 63) < 2.0;
  }
  if (!exact) {
    sp[lane] = pd;
    cum = 0;
    for (int j = 0; j < n8; j += 8) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const double t = sp[j + q];
        cum += j + q <= lane ? t : 0.0;
      }
    }
  }
  const double thr = P.min_p * readlane_f64(pd, 0);
  const unsigned long long minp = __ballot(lane > 0 && lane < n && pd < thr);
  const unsigned long long topp = __ballot(lane < n && cum >= P.top_p);
  const int f1 = minp ? (int)__ffsll((long long)minp) - 1 : n;   // break before adding f1
  const int f2 = topp ? (int)__ffsll((long long)topp) - 1 : n;   // break after adding f2
  const int cut = f1 <= f2 ? f1 : f2 + 1;
  // keptSum (src/sampler.ts:107-108) adds probs[0, cutoff) from 0 in the
  // same order as cumProb: it equals cumProb at cutoff - 1
  const double kept = readlane_f64(cum, cut - 1);
  const double r0 = u * kept;
  unsigned long long hit;
  if (exact) {
    hit = __ballot(lane < cut && cum >= r0);
  } else {
    double r = r0;   // r after subtracting index `lane`
    const int c8 = (cut + 7) & ~7;
    for (int j = 0; j < c8; j += 8) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const double t = sp[j + q];
        r -= j + q <= lane ? t : 0.0;
      }
    }
    hit = __ballot(lane < cut && r <= 0);
  }
  *cutoff = cut;
  return hit ? (int)__ffsll((long long)hit) - 1 : cut - 1;
}

// Completes a row of the row kernel in wave 0 from F, the row's top-64 list
// (sorted packed candidates, one per lane).  extra_ties: logits equal to the
// k-th largest may exist beyond F.  Replays the reference's slot scan when an
// equal-value group can change the token (or the candidate outputs), and
// always when force_replay (the candidate list overflowed).
// acquire_replay: other workgroups wrote parts of the row (split rows), so a
// replay first acquires their stores at agent scope.
// The tail's state between its decision and its outputs.
struct TailState {
  uint32_t key, T;
  int32_t id;
  int n, cut, pick;
  float prob;
  bool boundary_tie, internal_tie, need;
};

// The draw from F, and whether the slot replay is needed (need).
__device__ __forceinline__ TailState tail_decide(const LaunchArgs &a, const RowPlan &P,
                                                 unsigned long long F, bool extra_ties,
                                                 bool force_replay, double u, double *sp) {
  const int lane = lane_id();
  const int k = P.k;
  TailState st;
  const uint32_t fkey = cand_key(F);
  const unsigned long long Fk = __shfl(F, k - 1);
  st.T = cand_key(Fk);           // 0: fewer than k candidates
  const int n_sel = __popcll(__ballot(F != 0ull && fkey >= st.T));
  st.n = n_sel < k ? n_sel : k;
  st.boundary_tie = n_sel > k || (st.T != 0 && extra_ties);
  const uint32_t next_key = __shfl_down(fkey, 1);
  st.internal_tie = __ballot(lane + 1 < st.n && next_key == fkey) != 0;
  st.key = fkey;
  st.id = (int32_t)cand_idx(F);
  st.cut = 0;
  st.prob = 0.f;
  st.pick = force_replay ? -1 : wave_tail(st.key, st.n, P, u, &st.cut, &st.prob, sp);
  st.need = false;
  if (st.boundary_tie || st.internal_tie || force_replay) {
    // the order inside a group of equal values follows the slot history
    st.need = a.want_cands != 0 || force_replay;
    if (!st.need && st.pick >= 0) {
      const uint32_t kp = readlane_u32(st.key, st.pick);
      const uint32_t km = st.pick > 0 ? readlane_u32(st.key, st.pick - 1) : 0u;
      const uint32_t kn = st.pick + 1 < st.n ? readlane_u32(st.key, st.pick + 1) : 0u;
      st.need = (st.pick > 0 && km == kp) || (st.pick + 1 < st.n && kn == kp) ||
                (st.boundary_tie && kp == st.T);
    }
  }
  return st;
}

// The replay when needed, then the token and the optional outputs (RB:
// the replay's logits in flight per lane).
template <int RB = 16>
__device__ __forceinline__ void tail_finish(const LaunchArgs &a, const RowPlan &P, int row,
                                            const float *rowp, TailState st, double u,
                                            float *rsv, int32_t *rsid, double *sp,
                                            bool acquire_replay, const uint32_t *bkey,
                                            bool staged = false) {
  const int lane = lane_id();
  const int k = P.k;
  bool replayed = false;
  if (st.need) {
    if (!staged) {   // staged: replay_staged left the slots in rsv / rsid, in order
      if (acquire_replay) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      replay_row<RB>(rowp, a.vocab, k, rsv, rsid, bkey);
    }
    const bool filled = lane < k && rsid[lane] >= 0;
    unsigned long long x = filled ? pack_cand(f2key(rsv[lane]), (uint32_t)lane) : 0ull;
    // value descending, slot ascending (stable sort); the staged replay
    // stored its slots in that order already
    if (!staged) x = wave_sort_desc64(x);
    st.n = __popcll(__ballot(filled));
    st.key = cand_key(x);
    st.id = lane < st.n ? rsid[cand_idx(x)] : -1;
    st.pick = wave_tail(st.key, st.n, P, u, &st.cut, &st.prob, sp);
    replayed = true;
  }
  const int token = st.pick >= 0 ? __shfl(st.id, st.pick) : 0;
  if (lane == 0) {
    put_token(a, row, token);
    if (a.cand_count_out) a.cand_count_out[row] = st.n;
    if (a.cutoff_out) a.cutoff_out[row] = st.cut;
    if (a.row_flags) {
      uint32_t fl = 0;
      if (replayed) fl |= HS_ROW_REPLAYED;
      if (st.boundary_tie || st.internal_tie) fl |= HS_ROW_TIES;
      if (st.n < 2) fl |= HS_ROW_SINGLE;
      a.row_flags[row] = fl;
    }
  }
  const int cs = a.cand_stride;
  if (lane < st.n && lane < cs) {
    if (a.cand_ids) a.cand_ids[(int64_t)row * cs + lane] = st.id;
    if (a.cand_probs) a.cand_probs[(int64_t)row * cs + lane] = st.prob;
  }
}

template <int RB = 16>
__device__ __forceinline__ void finish_wave(const LaunchArgs &a, const RowPlan &P, int row, const float *rowp,
                            unsigned long long F, bool extra_ties, bool force_replay, double u,
                            float *rsv, int32_t *rsid, double *sp, bool acquire_replay = false) {
  const TailState st = tail_decide(a, P, F, extra_ties, force_replay, u, sp);
  tail_finish<RB>(a, P, row, rowp, st, u, rsv, rsid, sp, acquire_replay, nullptr);
}

size_t row_smem_bytes(int vocab) {
  const size_t words = ((size_t)vocab + 31) / 32;
  return (size_t)kRowCandCap * 8 + (size_t)kSortCap * 8 + 64 * 8 + (size_t)kSmallK * 8 +
         words * 4;
}

// ---- split rows: a part's hand-over
//
// A part publishes its list (candidates with global indices) and meta data
// with agent-scope stores, which write through to the point where every XCD
// sees them, waits until its own stores have completed, and only then counts
// itself in.  The part that counts S reads the others' data after an
// agent-scope acquire and completes the row; no workgroup ever waits for
// another.  The last part also resets the counter for the next call.
__device__ __forceinline__ void store_agent(unsigned long long *p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(int32_t *p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T load_agent(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Counts the calling part in (after its published stores completed); true
// in the part that completes the row.  That part reads what the others
// published with agent-scope loads, issued only after the count returned,
// so they observe every store completed before the others counted
// themselves in.  (No acquire fence: on this GPU it invalidates the XCD's
// L2, which stalls every workgroup there; plain loads of shared data need
// it, as before a replay of the row.)  `last` is LDS.  Every thread of the
// workgroup calls it.
__device__ __forceinline__ bool split_arrive(const Workspace &ws, int slot, int S, int32_t *last) {
  __builtin_amdgcn_s_waitcnt(0);   // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(ws.split_cnt + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last = old == (uint32_t)(S - 1);
    if (*last) store_agent(ws.split_cnt + slot, 0u);   // for the next call
  }
  __syncthreads();
  return *last != 0;
}

// Top 64 of two descending lists of 64 packed candidates (one per lane), by
// one wave: the elementwise maximum of a and b reversed is bitonic and holds
// the 64 largest, a half-cleaner cascade sorts it.  `disc` keeps the largest
// key left out (per lane).
__device__ __forceinline__ unsigned long long merge_top64(unsigned long long a, unsigned long long b,
                                                          uint32_t &disc) {
  const int lane = lane_id();
  const unsigned long long br = __shfl(b, 63 - lane);
  unsigned long long c = a > br ? a : br;
  const uint32_t dk = cand_key(a > br ? br : a);
  disc = dk > disc ? dk : disc;
#pragma unroll
  for (int j = 32; j >= 1; j >>= 1) {
    const unsigned long long o = __shfl_xor(c, j);
    c = (lane & j) ? (o < c ? o : c) : (o > c ? o : c);
  }
  return c;
}

// NT threads (tid: 0..NT-1, whole waves): bkey[b] = key of the largest logit
// of logits [64 b, 64 b + 64) of the row (0 when none is above -Infinity),
// for the slot replay to skip blocks.  A 16-lane DPP row takes one block, a
// float4 per lane.  In a 16-byte aligned row every read is a 16-byte load (8
// per thread in flight, 120-128 KiB per workgroup); otherwise 4 slots per
// thread are read by elements.
template <int NT>
__device__ void block_keys(const float *rowp, int V, uint32_t *bkey, int tid) {
  const int nf = ((V + 63) >> 6) * 16;   // float4 slots, 16 per block
  // the block maximum of each thread's slot key, by its DPP row (row_shr:1,
  // 2, 4, 8: lane 15 holds it)
  auto put = [&](int f, uint32_t x) {
    uint32_t y;
    y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x111, 0xF, 0xF, false); x = x > y ? x : y;
    y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x112, 0xF, 0xF, false); x = x > y ? x : y;
    y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x114, 0xF, 0xF, false); x = x > y ? x : y;
    y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x118, 0xF, 0xF, false); x = x > y ? x : y;
    if ((tid & 15) == 15 && f < nf) bkey[f >> 4] = x;
  };
  const int full = V >> 2;   // slots wholly inside the row
  if ((reinterpret_cast<uintptr_t>(rowp) & 15) == 0 && full > 0) {
    // every slot read as one float4 (clamped to the last whole one); the
    // slot holding the row's last logits (V % 4 of them) takes them one by
    // one, and slots past the row have key 0
    constexpr int UN = 8;
    const float4 *r4 = reinterpret_cast<const float4 *>(rowp);
    for (int f0 = 0; f0 < nf; f0 += UN * NT) {
      float4 v[UN];
#pragma unroll
      for (int u = 0; u < UN; ++u) v[u] = r4[min(f0 + u * NT + tid, full - 1)];
#pragma unroll
      for (int u = 0; u < UN; ++u) {
        const int f = f0 + u * NT + tid;
        uint32_t kk = 0;
        if (f < full) {
          const uint32_t a = max(f2key(v[u].x), f2key(v[u].y)), b = max(f2key(v[u].z), f2key(v[u].w));
          kk = max(a, b);
        } else if (f == full) {
          for (int e = 4 * f; e < V; ++e) kk = max(kk, f2key(rowp[e]));
        }
        put(f, kk);
      }
    }
    return;
  }
  int f0 = 0;
  constexpr int UT = 4;
  for (; f0 < nf; f0 += UT * NT) {
    // every read issued before any is used
    float v[UT][4];
#pragma unroll
    for (int u = 0; u < UT; ++u)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = 4 * (f0 + u * NT + tid) + q;
        v[u][q] = rowp[e < V ? e : 0];   // always a read inside the row
      }
#pragma unroll
    for (int u = 0; u < UT; ++u) {
      const int f = f0 + u * NT + tid;
      uint32_t kk = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t kv = 4 * f + q < V ? f2key(v[u][q]) : 0u;
        kk = kk > kv ? kk : kv;
      }
      put(f, kk);
    }
  }
}

struct RowSmem {
  SelectSmem sel;
  TailSmem tail;
  unsigned long long best[kRowWaves];
  uint32_t t_min, theta, key64;
  uint32_t theta2;             // refined bound, published by wave 0 mid-row
  int32_t wcnt[kRowWaves];     // candidates each wave has appended (published)
  int32_t n_l, n_f, ovf, done, last;
  int32_t tie;                 // wave 0's draw needs the slot replay
  int32_t pub[4];              // the staged replay's list length and end, per step parity
};

// SPLIT: a.split workgroups share a row, each streaming one part of it (a
// run of whole float4s) as if it were a row of its own; the last part to
// finish merges the parts' candidates and completes the row.
template <bool VEC, bool SPLIT>
__global__ __launch_bounds__(kRowThreads) void row_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long rdyn[];
  unsigned long long *cbuf = rdyn;                         // kRowCandCap candidates
  unsigned long long *srt = cbuf + kRowCandCap;            // kSortCap (fallback select)
  uint32_t *lmax = reinterpret_cast<uint32_t *>(srt);      // round-0 lane maxima (aliases srt)
  unsigned long long *top = srt + kSortCap;                // 64: sorted top of the row
  float *rsv = reinterpret_cast<float *>(top + 64);        // kSmallK replay slots
  int32_t *rsid = reinterpret_cast<int32_t *>(rsv + kSmallK);
  uint32_t *bitmap = reinterpret_cast<uint32_t *>(rsid + kSmallK);   // ceil(V/32)
  __shared__ RowSmem rs;

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform_i32(tid >> 6);
  int slot = (int)blockIdx.x, part = 0, eoff = 0, V = a.vocab;
  if (SPLIT) {   // this part: logits [eoff, eoff + V) of the row
    const int S = a.split;
    slot = (int)blockIdx.x / S;
    part = (int)blockIdx.x - slot * S;
    const int nf4 = (a.vocab + 3) >> 2, per = (nf4 + S - 1) / S;
    const int f0 = min(nf4, part * per), f1 = min(nf4, f0 + per);
    eoff = 4 * f0;
    V = min(a.vocab, 4 * f1) - eoff;
  }
  const int row = a.rows_direct ? slot : ws.row_list[slot];
  float *const rowfull = a.logits + (int64_t)row * a.stride;
  float *rowp = rowfull + eoff;
  const int nr = row_rounds(V);

  // Round 0 is requested first; the last <= 128 history ids (one per thread
  // of waves 0-1; their offsets come through the scalar cache) right after
  // it, so that they arrive with round 0 (a wave's reads complete in order);
  // then round 1.  Round 2 follows as soon as round 0 has arrived, so the
  // bound below is computed while rounds 1 and 2 stream.
  RowSrc src;
  src.lim = VEC ? (V & ~3) : V;
  src.x4 = make_rsrc(rowp, 4u * (uint32_t)(V & ~3));
  src.x1 = make_rsrc(rowp, 4u * (uint32_t)V);
  float v0[kR0NV][4], va[kRowNV][4], vb[kRowNV][4];
  load_rd<kR0NV, VEC>(v0, src, 0, tid);
  __builtin_amdgcn_sched_barrier(0);
  const HistTail ht = hist_tail(a, row, tid);
  const int hraw = ht.id, hist_n = ht.n;
  __builtin_amdgcn_sched_barrier(0);
  load_rd<kRowNV, VEC>(vb, src, round_base(1), tid);   // past the row when nr == 1
  // the logits past the last whole float4 (VEC only), read by thread 0
  float tl[3] = {0.f, 0.f, 0.f};
  if (VEC) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int e = src.lim + q;
      tl[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          src.x1, (tid == 0 && e < V ? e : V) * 4, 0, 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // the row's plan through the scalar cache, which does not queue behind
  // the vector loads
  const RowPlan *plan = ws.plans + row;
  const int mode = load_scalar(&plan->mode);
  const int k = load_scalar(&plan->k);
  const int penbits = load_scalar(&plan->pen);
  const double prep = load_scalar(&plan->rep);
  const double temperature = load_scalar(&plan->temperature);
  const double top_p = load_scalar(&plan->top_p), min_p = load_scalar(&plan->min_p);
  const double u = load_scalar(a.uniforms + row);

  const bool greedy = mode == kModeGreedy;
  // presence / frequency rows were penalised in place by pen_kernel
  const bool rep = (penbits & kPenRep) && !(penbits & kPenPF);
  if (tid == 0) {
    rs.t_min = 0xFFFFFFFFu; rs.theta = 0; rs.theta2 = 0; rs.key64 = 0;
    rs.n_l = 0; rs.n_f = 0; rs.ovf = 0; rs.done = 0;
  }
  if (tid < kRowWaves) rs.wcnt[tid] = 0;
  if (tid < 64) top[tid] = 0ull;
  // this wave's segment of the candidate list and its count (wave-uniform)
  unsigned long long *seg = cbuf + wave * kSegCap;
  int cnt = 0;
  auto publish = [&]() {
    if (lane == 0) __atomic_store_n(&rs.wcnt[wave], cnt, __ATOMIC_RELAXED);
  };

  // src/sampler.ts:24-33: the distinct ids of the last 128 history entries.
  // Their logits leave the stream (bitmap); the thread holding the first
  // occurrence of an id keeps its raw logit for the end of the row.
  int pid = -1;
  if (rep) {
    const int words = (V + 31) >> 5;
    for (int i = tid; i < words; i += kRowThreads) bitmap[i] = 0;
    __syncthreads();
    const int hid = tid < hist_n ? hraw - eoff : -1;   // relative to the part
    if (hid >= 0 && hid < V) {
      const uint32_t bit = 1u << (hid & 31);
      if (!(atomicOr(&bitmap[hid >> 5], bit) & bit)) pid = hid;   // the first occurrence owns the id
    }
  }
  // the owner's raw logit, used after the stream (its latency hides behind it)
  const float pval =
      __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(src.x1, (pid >= 0 ? pid : V) * 4, 0, 0));
  __syncthreads();   // bitmap complete, LDS cleared

  // ---- round 0 fixes the bound: theta = the exact k-th largest of the 1024
  // lane maxima (each a distinct logit outside the repetition set), a lower
  // bound of the row's k-th largest value
  clip_rd<kR0NV>(v0, 0, tid, src.lim);
  if (rep) mask_penalised<kR0NV>(v0, 0, tid, V, bitmap);
  unsigned long long best = 0;   // greedy: packed maximum
  uint32_t key = 0;              // lane maximum of round 0
  if (greedy)
    best = greedy_rd<kR0NV>(v0, 0, tid, best);
  else
    key = f2key(rd_max<kR0NV>(v0));
  __builtin_amdgcn_sched_barrier(0);
  load_rd<kRowNV, VEC>(va, src, round_base(2), tid);
  __builtin_amdgcn_sched_barrier(0);
  float xf = -FLT_MAX;
  uint32_t theta = 0;
  if (!greedy) {
    // Each wave's j-th largest lane maximum, j = ceil(k/16): the 16 waves
    // together hold at least 16j >= k lanes at or above the smallest of them.
    const uint32_t mj = wave_jth_largest(key, (k + kRowWaves - 1) / kRowWaves);
    if (lane == 0) atomicMin(&rs.t_min, mj);   // 0 when a wave has fewer such lanes
    __syncthreads();
    const uint32_t lo0 = (uint32_t)uniform_i32((int)rs.t_min);
    const uint32_t lo = lo0 ? lo0 : 1u;
    const bool pass = key >= lo;
    const unsigned long long b = __ballot(pass);
    if (b) {
      const int leader = __ffsll((long long)b) - 1;
      int bp = 0;
      if (lane == leader) bp = atomicAdd(&rs.n_l, __popcll(b));
      bp = __shfl(bp, leader);
      if (pass) lmax[bp + (int)lanes_below(b)] = key;
    }
    __syncthreads();
    if (wave == 0) {
      const uint32_t th = wave_kth_of_list(lmax, rs.n_l, k, lo);
      if (lane == 0) rs.theta = th;
    }
    __syncthreads();
    theta = (uint32_t)uniform_i32((int)rs.theta);
    xf = key_floor(theta ? theta : 1u);
    append_rd<kR0NV>(v0, 0, tid, xf, seg, cnt);   // masked already
    publish();
  }

  // ---- rounds >= 1: candidates are rare.  vb holds the odd rounds, va the
  // even ones.
  for (int r = 1; r < nr; r += 2) {
    if (!greedy) {
      if (r == 3 && wave == 0) {
        // Wave 0 alone tightens the bound to the exact k-th largest of the
        // candidates published so far; the other waves pick it up at their
        // next round.  Any k of the row's logits outside the repetition set
        // bound its k-th largest.
        const uint32_t t2 = wave_snapshot_bound(cbuf, rs.wcnt, k, theta, bitmap, rep);
        if (lane == 0 && t2 > theta) __atomic_store_n(&rs.theta2, t2, __ATOMIC_RELAXED);
      }
      const uint32_t t2 =
          (uint32_t)uniform_i32((int)__atomic_load_n(&rs.theta2, __ATOMIC_RELAXED));
      if (t2 > theta) { theta = t2; xf = key_floor(theta); }
    }
    clip_rd<kRowNV>(vb, round_base(r), tid, src.lim);
    if (greedy) {
      if (rep) mask_penalised<kRowNV>(vb, round_base(r), tid, V, bitmap);
      best = greedy_rd<kRowNV>(vb, round_base(r), tid, best);
    } else {
      append_rd<kRowNV>(vb, round_base(r), tid, xf, seg, cnt);
      publish();
    }
    load_rd<kRowNV, VEC>(vb, src, round_base(r + 2), tid);   // past the row near its end
    if (r + 1 >= nr) break;
    clip_rd<kRowNV>(va, round_base(r + 1), tid, src.lim);
    if (greedy) {
      if (rep) mask_penalised<kRowNV>(va, round_base(r + 1), tid, V, bitmap);
      best = greedy_rd<kRowNV>(va, round_base(r + 1), tid, best);
    } else {
      append_rd<kRowNV>(va, round_base(r + 1), tid, xf, seg, cnt);
      publish();
    }
    load_rd<kRowNV, VEC>(va, src, round_base(r + 3), tid);
  }

  // The penalised logits go back in place.  No barrier is needed first:
  // whatever a wave still streaming reads at these ids is left out (masked,
  // or dropped with the repetition set at the end).
  float pv = 0.f;
  if (pid >= 0) {
    RowPlan pr;
    pr.rep = prep;
    pr.pen = kPenRep;
    pv = penalise(pval, true, 0u, pr);
    if (SPLIT)
      store_agent(rowp + pid, pv);   // read by the part that completes the row
    else
      rowp[pid] = pv;
  }

  // the tail logits (thread 0) outside the repetition set
  bool tail_ok[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int e = src.lim + q;
    tail_ok[q] = VEC && tid == 0 && e < V && !(rep && ((bitmap[e >> 5] >> (e & 31)) & 1u));
  }

  if (greedy) {
    if (pid >= 0) {
      const uint32_t key = f2key(pv);
      const unsigned long long c = key ? pack_cand(key, (uint32_t)pid) : 0ull;
      best = c > best ? c : best;
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const uint32_t key = tail_ok[q] ? f2key(tl[q]) : 0u;
      const unsigned long long c = key ? pack_cand(key, (uint32_t)(src.lim + q)) : 0ull;
      best = c > best ? c : best;
    }
    best = wave_max64(best);
    if (lane == 0) rs.best[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long bb = rs.best[0];
      for (int w = 1; w < kRowWaves; ++w) bb = rs.best[w] > bb ? rs.best[w] : bb;
      if (SPLIT)   // the same packed form with the row's index (no borrow: idx + eoff < 2^32)
        store_agent(&ws.split_meta[blockIdx.x].best, bb ? bb - (unsigned long long)eoff : 0ull);
      else
        write_greedy(a, row, rowp[0], bb);
    }
    if (SPLIT && split_arrive(ws, slot, a.split, &rs.last) && tid == 0) {
      unsigned long long bb = 0;
      for (int p = 0; p < a.split; ++p) {
        const unsigned long long b = load_agent(&ws.split_meta[slot * a.split + p].best);
        bb = b > bb ? b : bb;
      }
      write_greedy(a, row, load_agent(rowfull), bb);
    }
    return;
  }

  // The first wave to end its stream tightens the bound once more, from the
  // entries published so far (every wave has published all but at most its
  // last round).  After the barrier every wave moves into srt the entries of
  // its segment at or above the final bound, leaving out the raw logits of
  // the repetition set, and its penalised and tail logits at or above it.
  {
    int first = 0;
    if (lane == 0) first = atomicAdd(&rs.done, 1) == 0;
    if (uniform_i32(first)) {
      const uint32_t t0 = (uint32_t)uniform_i32((int)__atomic_load_n(&rs.theta2, __ATOMIC_RELAXED));
      const uint32_t cur = t0 > theta ? t0 : theta;
      const uint32_t t2 = wave_snapshot_bound(cbuf, rs.wcnt, k, cur, bitmap, rep);
      if (lane == 0 && t2 > cur) atomicMax(&rs.theta2, t2);
    }
  }
  __syncthreads();
  {
    const uint32_t t2 = (uint32_t)uniform_i32((int)rs.theta2);
    if (t2 > theta) theta = t2;
  }
  const uint32_t lo = theta ? theta : 1u;
  xf = key_floor(lo);
  auto join = [&](bool pass, unsigned long long c) {
    const unsigned long long b = __ballot(pass);
    if (b) {
      const int leader = __ffsll((long long)b) - 1;
      int bp = 0;
      if (lane == leader) bp = atomicAdd(&rs.n_f, __popcll(b));
      bp = __shfl(bp, leader);
      const int p = bp + (int)lanes_below(b);
      if (pass && p < kSortCap) srt[p] = c;
    }
  };
  if (cnt > kSegCap) {   // the segment filled up and lost candidates: replay the row
    if (lane == 0) rs.ovf = 1;
  } else {
    for (int i = lane; i < cnt; i += 64) {
      const unsigned long long c = seg[i];
      const uint32_t id = cand_idx(c);
      join(cand_key(c) >= lo && !(rep && ((bitmap[id >> 5] >> (id & 31)) & 1u)), c);
    }
  }
  join(pid >= 0 && pv >= xf, pack_cand(f2key(pv), (uint32_t)pid));
  if (VEC && src.lim < V) {
#pragma unroll
    for (int q = 0; q < 3; ++q)
      join(tail_ok[q] && tl[q] >= xf, pack_cand(f2key(tl[q]), (uint32_t)(src.lim + q)));
  }
  __syncthreads();
  const int n_all = rs.n_f;
  bool overflow = rs.ovf != 0 || n_all > kSortCap;
  unsigned long long F = 0;
  bool extra = false;
  if (SPLIT) {
    // The part hands over its top 64 (every logit of the row's top k, k <= 64,
    // is among the top k of its part) and the key of its 65th, which flags
    // values equal to the row's k-th largest left out of the list.
    const int S = a.split;
    overflow = overflow || n_all > kRowThreads;   // ties beyond the ranking's reach: replay
    if (!overflow) rank_top64(srt, n_all, top, &rs.key64);
    if (wave == 0) {
      SplitMeta *m = ws.split_meta + blockIdx.x;
      const unsigned long long c = top[lane];
      if (!overflow && lane < n_all)
        store_agent(ws.split_list + (int64_t)blockIdx.x * kPartCap + lane, c - (unsigned long long)eoff);
      if (lane == 0) {
        store_agent(&m->count, overflow ? -1 : min(n_all, kPartCap));
        store_agent(&m->theta, lo);
        store_agent(&m->key64, rs.key64);
      }
    }
    if (!split_arrive(ws, slot, S, &rs.last)) return;
    // The last part: the top 64 of the union of the parts' lists, by a tree
    // of pairwise merges (wave w merges lists 2w and 2w + 1).  The parts'
    // meta data and the first level's lists are requested together.
    const SplitMeta *m0 = ws.split_meta + (int64_t)slot * S;
    const unsigned long long *l0 = ws.split_list + (int64_t)slot * S * kPartCap;
    int cntp = 0;
    uint32_t k64 = 0;
    if (lane < S) {
      cntp = load_agent(&m0[lane].count);
      k64 = load_agent(&m0[lane].key64);
    }
    unsigned long long ea = 0, eb = 0;
    if (2 * wave < S) ea = load_agent(l0 + (2 * wave) * kPartCap + lane);
    if (2 * wave + 1 < S) eb = load_agent(l0 + (2 * wave + 1) * kPartCap + lane);
    overflow = __ballot(cntp < 0) != 0;   // a part's list is incomplete: replay
    if (lane >= __shfl(cntp, (2 * wave) & 63)) ea = 0ull;        // entries past a count are stale
    if (lane >= __shfl(cntp, (2 * wave + 1) & 63)) eb = 0ull;
    uint32_t disc = 0;
    unsigned long long c = 0;
    int L = (S + 1) / 2;   // lists after this level
    if (2 * wave < S) c = merge_top64(ea, eb, disc);
    for (int lvl = 0; L > 1; ++lvl) {
      unsigned long long *buf = srt + (lvl & 1) * (kSortCap / 2);   // 16 lists of 64 each
      if (wave < L) buf[wave * 64 + lane] = c;
      __syncthreads();
      const int L2 = (L + 1) / 2;
      if (wave < L2) {
        const unsigned long long x = buf[(2 * wave) * 64 + lane];
        const unsigned long long y = 2 * wave + 1 < L ? buf[(2 * wave + 1) * 64 + lane] : 0ull;
        c = merge_top64(x, y, disc);
      }
      L = L2;
    }
    disc = wave_max_u32(disc);
    if (tid == 0) rs.key64 = 0;
    __syncthreads();
    if (lane == 0 && disc) atomicMax(&rs.key64, disc);
    __syncthreads();
    RowPlan P;
    P.temperature = temperature;
    P.top_p = top_p;
    P.min_p = min_p;
    P.k = k;
    // Wave 0 draws; when the slot replay is needed, the whole workgroup
    // first records the largest logit of every 64-logit block of the row, as
    // for a whole row, after acquiring the other parts' penalised write-backs
    // at agent scope.  The other waves wait for the decision.
    TailState st;
    if (wave == 0) {
      if (!overflow) {
        F = c;
        const uint32_t Tk = cand_key(__shfl(F, k - 1));
        // the union's 65th, or a part's own 65th, equal to the row's k-th
        // largest: more values equal to it may exist beyond F
        extra = Tk != 0u && (rs.key64 == Tk || __ballot(lane < S && k64 == Tk) != 0);
      }
      st = tail_decide(a, P, F, extra, overflow, u, reinterpret_cast<double *>(top));
      if (lane == 0) rs.tie = st.need ? 1 : 0;
    }
    __syncthreads();
    const uint32_t *bkey = nullptr;
    bool staged = false;
    if (rs.tie) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      // as for a whole row: the first k blocks copied into LDS, replayed by
      // wave 0 while the others take the block keys
      PackedSlots ls(k);
      const int h0 = min(min(k, (a.vocab + 63) >> 6), kHeadBlocks);
      uint32_t *ring = reinterpret_cast<uint32_t *>(srt), *hkeys = ring + kReplayRing;
      replay_head_keys<kRowThreads>(rowfull, a.vocab, h0, hkeys);
      __syncthreads();
      if (wave == 0)
        ls.scan_keys(hkeys, h0);
      else
        block_keys<kRowThreads - 64>(rowfull, a.vocab, reinterpret_cast<uint32_t *>(cbuf), tid - 64);
      __syncthreads();
      bkey = reinterpret_cast<const uint32_t *>(cbuf);
      staged = replay_staged<kRowThreads>(rowfull, a.vocab, k, ls, h0,
                                          reinterpret_cast<uint32_t *>(cbuf), 2 * kRowCandCap, ring,
                                          kReplayRing, rs.pub, rsv, rsid);
    }
    if (wave != 0) return;
    tail_finish(a, P, row, rowfull, st, u, rsv, rsid, reinterpret_cast<double *>(top), true, bkey,
                staged);
    return;
  }
  if (!overflow && n_all <= kRowThreads) {
    rank_top64(srt, n_all, top, &rs.key64);
    if (wave == 0) {
      F = top[lane];
      const uint32_t Tk = cand_key(__shfl(F, k - 1));
      extra = rs.key64 != 0u && rs.key64 == Tk;
    }
  } else if (!overflow) {
    // rare: many candidates reach the bound (ties); select block-wide first,
    // from srt into cbuf (the segments are no longer needed)
    const SelResult sel = select_into<kRowThreads>(
        n_all, [srt](int p) { return srt[p]; }, 1u, k, cbuf, rs.sel, rs.tail);
    const int n_sel = sel.n_sel;
    if (n_sel < 0) overflow = true;
    if (wave == 0 && !overflow) {
      F = lane < n_sel ? cbuf[lane] : 0ull;
      extra = n_sel > 64;
    }
  }
  // Wave 0 draws; when an equal-value group makes the reference's slot
  // replay necessary, the whole block first records the largest logit of
  // every 64-logit block of the row (into cbuf, read into F already), so that
  // the replay, by wave 0 alone, reads only the blocks that can hold an
  // entering logit.  The other waves wait for the decision.
  RowPlan P;
  P.temperature = temperature;
  P.top_p = top_p;
  P.min_p = min_p;
  P.k = k;
  TailState st;
  if (wave == 0) {
    st = tail_decide(a, P, F, extra, overflow, u, reinterpret_cast<double *>(top));
    if (lane == 0) rs.tie = st.need ? 1 : 0;
  }
  __syncthreads();
  const uint32_t *bkey = nullptr;
  bool staged = false;
  if (rs.tie) {
    // the first k blocks (the slots fill there and most of the row's
    // entering logits lie there) are copied into LDS, and wave 0 replays them
    // while the others take the block keys; then the staged replay of the
    // blocks listed after them
    PackedSlots ls(k);
    const int h0 = min(min(k, (V + 63) >> 6), kHeadBlocks);
    uint32_t *ring = reinterpret_cast<uint32_t *>(srt), *hkeys = ring + kReplayRing;
    replay_head_keys<kRowThreads>(rowp, V, h0, hkeys);
    __syncthreads();
    if (wave == 0)
      ls.scan_keys(hkeys, h0);
    else
      block_keys<kRowThreads - 64>(rowp, V, reinterpret_cast<uint32_t *>(cbuf), tid - 64);
    __syncthreads();
    bkey = reinterpret_cast<const uint32_t *>(cbuf);
    staged = replay_staged<kRowThreads>(rowp, V, k, ls, h0, reinterpret_cast<uint32_t *>(cbuf),
                                        2 * kRowCandCap, ring, kReplayRing, rs.pub, rsv, rsid);
  }
  if (wave != 0) return;
  tail_finish(a, P, row, rowp, st, u, rsv, rsid, reinterpret_cast<double *>(top), false, bkey,
              staged);
}

// ---------------------------------------------------------------- mid kernel

// Rows with 64 < k <= 1024: the row kernel's stream, with the bound taken
// from an LDS histogram of keys (kMidBins bins of the top key bits).  Round 0
// is counted whole; from then on only the logits at or above the bound are
// counted (they are the candidates), which keeps every bin at or above any
// later bound exact.  Each wave recomputes the bound from the histogram at
// every round and drops the entries of its segment that fell below it.  At
// the end the candidates at or above the final bound (about k plus one bin)
// are sorted and finish_row completes the row.

// Turns a round into keys and counts every finite one; returns the largest.
template <int NV>
__device__ __forceinline__ uint32_t hist_keys(const float (&v)[NV][4], uint32_t (&kk)[NV][4],
                                              uint32_t *hist) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t key = f2key(v[j][q]);
      kk[j][q] = key;
      if (key) atomicAdd(&hist[key >> kMidShift], 1u);
      m = key > m ? key : m;
    }
  return m;
}

// Appends every key >= lo (lo >= 1) of a round to the wave's segment.
template <int NV>
__device__ __forceinline__ void append_keys(const uint32_t (&kk)[NV][4], int fb, int tid,
                                            uint32_t lo, unsigned long long *seg, int &cnt) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t mx = max(max(kk[j][0], kk[j][1]), max(kk[j][2], kk[j][3]));
    if (!__ballot(mx >= lo)) continue;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool pass = kk[j][q] >= lo;
      const unsigned long long b = __ballot(pass);
      if (b) {
        const int p = cnt + (int)lanes_below(b);
        if (pass && p < kSegCap)
          seg[p] = pack_cand(kk[j][q], (uint32_t)(slot_elem(fb, tid, j) + q));
        cnt = uniform_i32(cnt + __popcll(b));
      }
    }
  }
}

// append_rd that also counts every appended logit; returns the largest key
// appended.  The round's logits >= xf go to the segment as they pass (their
// value bits in place of the key); the keys, the bins and the maximum are
// then computed over the entries the round appended with every lane busy,
// where a row of many candidates would otherwise run that work per
// component with one or two lanes active.  (Entries past kSegCap are not
// counted: the counts stay lower bounds, and such a segment loses the row.)
template <int NV>
__device__ __forceinline__ uint32_t append_hist_rd(const float (&v)[NV][4], int fb, int tid, float xf,
                                                   unsigned long long *seg, int &cnt,
                                                   uint32_t *hist) {
  const int c0 = cnt;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float mx = fmaxf(fmaxf(v[j][0], v[j][1]), fmaxf(v[j][2], v[j][3]));
    if (!__builtin_amdgcn_ballot_w64(mx >= xf)) continue;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const unsigned long long b = __builtin_amdgcn_ballot_w64(v[j][q] >= xf);
      if (b) {
        const int p = cnt + (int)lanes_below(b);
        if (v[j][q] >= xf && p < kSegCap)
          seg[p] = ((unsigned long long)__float_as_uint(v[j][q]) << 32) |
                   (uint32_t)pack_cand(0u, (uint32_t)(slot_elem(fb, tid, j) + q));
        cnt = uniform_i32(cnt + __popcll(b));
      }
    }
  }
  // (a wave's LDS operations take effect in issue order)
  uint32_t m = 0;
  const int c1 = cnt < kSegCap ? cnt : kSegCap;
  for (int i = c0 + lane_id(); i < c1; i += 64) {
    const unsigned long long e = seg[i];
    const uint32_t key = f2key(__uint_as_float((uint32_t)(e >> 32)));
    seg[i] = ((unsigned long long)key << 32) | (uint32_t)e;
    atomicAdd(&hist[key >> kMidShift], 1u);
    m = key > m ? key : m;
  }
  return m;
}

// The largest bin edge t with at least k counted keys >= t, searching down
// from the bin of `top` (the largest counted key); 0 when fewer than k are
// counted.  Counts read while other waves still add are lower bounds of the
// final ones, so the result is a lower bound of the row's k-th largest.  A
// bin may hold a negative count (a left-out logit taken out before the
// stream counts it, or never counted): counts stay lower bounds, read as
// signed.
__device__ __forceinline__ uint32_t hist_bound(const uint32_t *hist, uint32_t top, int k) {
  const int lane = lane_id();
  int cum = 0;
  for (int base = (int)(top >> kMidShift); base >= 0; base -= 64) {
    const int b = base - lane;
    const uint32_t c = b >= 0 ? __atomic_load_n(hist + b, __ATOMIC_RELAXED) : 0u;
    const int incl = (int)wave_scan_incl(c);   // lane 0 holds the highest bin
    const int tot = (int)readlane_u32((uint32_t)incl, 63);
    if (cum + tot >= k) {
      const unsigned long long mk = __ballot(cum + incl >= k);
      const int L = __ffsll((long long)mk) - 1;
      return (uint32_t)(base - L) << kMidShift;
    }
    cum += tot;
  }
  return 0u;
}

// Drops the stored entries of a segment below lo (in place, order kept).
__device__ __forceinline__ void compact_seg(unsigned long long *seg, int &cnt, uint32_t lo) {
  const int lane = lane_id();
  const int n = cnt < kSegCap ? cnt : kSegCap;
  int m = 0;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const unsigned long long c = i < n ? seg[i] : 0ull;
    const bool keep = i < n && cand_key(c) >= lo;
    const unsigned long long b = __ballot(keep);
    if (keep) seg[m + (int)lanes_below(b)] = c;   // m <= base: entries not yet read stay
    m += __popcll(b);
  }
  cnt = uniform_i32(m);
}

// One round of the mid kernel: the bound from the histogram (dropping the
// segment's entries below it when it rose), then the round's candidates.
__device__ __forceinline__ void mid_step(float (&v)[kRowNV][4], int fb, int tid, int lim,
                                         int k, uint32_t *hist, uint32_t *top_key,
                                         unsigned long long *seg, int &cnt, uint32_t &theta,
                                         float &xf, bool &lost) {
  const uint32_t t =
      hist_bound(hist, (uint32_t)uniform_i32((int)__atomic_load_n(top_key, __ATOMIC_RELAXED)), k);
  if (t > theta) {
    theta = t;
    xf = key_floor(theta);
    lost = lost || cnt > kSegCap;
    compact_seg(seg, cnt, theta);
  }
  clip_rd<kRowNV>(v, fb, tid, lim);
  const uint32_t m = wave_max_u32(append_hist_rd<kRowNV>(v, fb, tid, xf, seg, cnt, hist));
  if ((tid & 63) == 0 && m) atomicMax(top_key, m);
}

// the penalty prologue's table and range buffer fit below the bitmap
static_assert((size_t)kRowCandCap * 8 + (size_t)kSortCap * 8 + (size_t)kMidBins * 4 >=
                  (size_t)kPenSlots * 8 &&
              (size_t)kRowCandCap * 8 + (size_t)kSortCap * 8 + (size_t)kMidBins * 4 >=
                  (size_t)(kPenRange + kPenRange / 32) * 4,
              "mid kernel LDS too small for the penalty prologue");

// The mid kernel's LDS: the stream's arrays, the bitmap, then the early list
// of a presence / frequency row (ids and values, 8 bytes each) in what remains
// of kMidLdsMax, at most kMidEarly.
__host__ __device__ __forceinline__ size_t mid_base_bytes(int vocab) {
  const size_t words = ((size_t)vocab + 31) / 32;
  return (size_t)kRowCandCap * 8 + (size_t)kSortCap * 8 + (size_t)kMidBins * 4 + words * 4;
}
__host__ __device__ __forceinline__ int mid_early_cap(int vocab) {
  const size_t base = mid_base_bytes(vocab);
  const size_t fit = base < (size_t)kMidLdsMax ? ((size_t)kMidLdsMax - base) / 8 : 0;
  return (int)(fit < (size_t)kMidEarly ? fit : (size_t)kMidEarly);
}
static_assert((size_t)kRowCandCap * 8 + (size_t)kSortCap * 8 + (size_t)kMidBins * 4 +
                      (size_t)kRowMaxVocab / 8 <= (size_t)kMidLdsMax,
              "mid kernel LDS");

size_t mid_smem_bytes(int vocab) { return mid_base_bytes(vocab) + 8 * (size_t)mid_early_cap(vocab); }

struct MidSmem {
  TailSmem tail;
  uint32_t top_key;
  int32_t n_f, ovf, n_sel, pen_full;
  float tl[3];   // the tail logits (VEC)
};

template <bool VEC>
__global__ __launch_bounds__(kRowThreads) void mid_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long mdyn[];
  unsigned long long *cbuf = mdyn;                                  // kRowCandCap
  unsigned long long *srt = cbuf + kRowCandCap;                     // kSortCap
  uint32_t *hist = reinterpret_cast<uint32_t *>(srt + kSortCap);    // kMidBins
  uint32_t *bitmap = hist + kMidBins;                               // ceil(V/32)
  __shared__ MidSmem ms;

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform_i32(tid >> 6);
  const int row = ws.mid_list[blockIdx.x];
  float *rowp = a.logits + (int64_t)row * a.stride;
  const int V = a.vocab;
  const int nr = row_rounds(V);

  const RowPlan *plan = ws.plans + row;
  const int penbits = load_scalar(&plan->pen);
  const bool pf = (penbits & kPenPF) != 0;
  // the penalties' part of the plan, by scalar reads (a vector read issued
  // after the rounds' reads would wait for them)
  RowPlan pp{};
  pp.pen = penbits;
  pp.rep = load_scalar(&plan->rep);
  pp.pres = load_scalar(&plan->pres);
  pp.freq = load_scalar(&plan->freq);

  // Reads in this order: a presence / frequency row's first history ids, the
  // repetition set's ids, the tail logits, rounds 0 and 1 (a wait for one
  // read waits for the reads before it, not after).
  const HistRow hrow = hist_row(a, row);
  int pids[4] = {-1, -1, -1, -1};
  if (pf) pen_request<kRowThreads>(hrow, pen_start(hrow, pp), pids);
  const HistTail ht = pf ? HistTail{-1, 0} : hist_tail(a, row, tid);
  const int hraw = ht.id, hist_n = ht.n;
  RowSrc src;
  src.lim = VEC ? (V & ~3) : V;
  src.x4 = make_rsrc(rowp, 4u * (uint32_t)(V & ~3));
  src.x1 = make_rsrc(rowp, 4u * (uint32_t)V);
  // the fewer than four logits past the last whole float4 (thread 0), kept
  // in LDS once they arrive
  float tl[3] = {0.f, 0.f, 0.f};
  auto load_tail = [&]() {
    if (VEC) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const int e = src.lim + q;
        tl[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            src.x1, (tid == 0 && e < V ? e : V) * 4, 0, 0));
      }
    }
  };
  load_tail();
  float v0[kR0NV][4], va[kRowNV][4], vb[kRowNV][4];
  load_rd<kR0NV, VEC>(v0, src, 0, tid);
  load_rd<kRowNV, VEC>(vb, src, round_base(1), tid);
  __builtin_amdgcn_sched_barrier(0);

  const int k = load_scalar(&plan->k);
  const int words = (V + 31) >> 5;
  const int ecap = mid_early_cap(V);
  int32_t *eid = reinterpret_cast<int32_t *>(bitmap + words);   // the penalised ids, and
  uint32_t *eaux = reinterpret_cast<uint32_t *>(eid + ecap);     //   their count words, then values
  __shared__ int32_t n_early;
  int ne = 0;                    // penalised ids listed
  float praw[2] = {0.f, 0.f};    // logits of list entries tid and tid + kRowThreads
  static_assert(kMidEarly <= 2 * kRowThreads, "two list entries per thread");

  // Presence / frequency rows: the row's distinct history ids are counted as
  // pen_kernel counts them, in the LDS the stream has not taken yet (the
  // candidate, sort and histogram arrays hold pen_smem_bytes()), while rounds
  // 0 and 1 are in flight, into a list (eid: id, eaux: count | rep bit 31)
  // and the bitmap.  The stream leaves the listed ids out; their logits are
  // requested now and needed only at the end of the row, where their
  // penalties are applied, stored in place and joined.  A row whose ids do
  // not fit the table or the list is rewritten in place now, waits for its
  // stores and reads rounds 0 and 1 again, unmasked.
  if (pf) {
    for (int i = tid; i < words; i += kRowThreads) bitmap[i] = 0u;
    if (tid == 0) n_early = 0;
    __syncthreads();
    auto slot = [&](int id, uint32_t cw) {
      const int p = atomicAdd(&n_early, 1);
      if (p < ecap) {
        eid[p] = id;
        eaux[p] = cw;
      }
      atomicOr(&bitmap[id >> 5], 1u << (id & 31));
    };
    const bool deferred = pen_row<kRowThreads, true>(
        hrow, pp, rowp, V, reinterpret_cast<uint32_t *>(mdyn), ms.pen_full, PenNoHook{}, &pids,
        slot);
    __syncthreads();   // the list and the bitmap are complete
    ne = n_early;
    if (!deferred || ne > ecap) {   // (uniform)
      if (deferred) pen_apply<kRowThreads>(reinterpret_cast<const uint32_t *>(mdyn), pp, rowp);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __syncthreads();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      load_tail();
      load_rd<kR0NV, VEC>(v0, src, 0, tid);
      load_rd<kRowNV, VEC>(vb, src, round_base(1), tid);
      ne = 0;
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int i = tid + c * kRowThreads;
        const int id = i < ne ? eid[i] : V;   // (past the row: 0, no read)
        praw[c] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(src.x1, id * 4, 0, 0));
      }
    }
  }
  // the ids the stream leaves out: the repetition set (rows without presence
  // / frequency), or a presence / frequency row's penalised ids
  const bool rep = (penbits & kPenRep) && !pf;
  const bool mask = rep || ne > 0;
  if (tid == 0) { ms.top_key = 0; ms.n_f = 0; ms.ovf = 0; ms.n_sel = 0; }
  for (int i = tid; i < kMidBins; i += kRowThreads) hist[i] = 0;
  unsigned long long *seg = cbuf + wave * kSegCap;
  int cnt = 0;
  bool lost = false;

  int pid = -1;
  if (rep) {
    for (int i = tid; i < words; i += kRowThreads) bitmap[i] = 0;
    __syncthreads();
    const int hid = tid < hist_n ? hraw : -1;
    if (hid >= 0 && hid < V) {
      const uint32_t bit = 1u << (hid & 31);
      if (!(atomicOr(&bitmap[hid >> 5], bit) & bit)) pid = hid;
    }
  }
  const float pval =
      __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(src.x1, (pid >= 0 ? pid : V) * 4, 0, 0));
  __syncthreads();   // bitmap complete, histogram cleared

  // ---- round 0 is counted whole; the bound follows from the histogram
  clip_rd<kR0NV>(v0, 0, tid, src.lim);
  if (mask) mask_penalised<kR0NV>(v0, 0, tid, V, bitmap);
  uint32_t k0[kR0NV][4];
  {
    const uint32_t m0 = wave_max_u32(hist_keys<kR0NV>(v0, k0, hist));
    if (lane == 0) atomicMax(&ms.top_key, m0);
  }
  __builtin_amdgcn_sched_barrier(0);
  load_rd<kRowNV, VEC>(va, src, round_base(2), tid);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();   // round 0 counted
  // the tail logits, kept in LDS until the end (their reads, issued before
  // round 0's, are done: no wait)
  if (VEC && tid == 0) {
#pragma unroll
    for (int q = 0; q < 3; ++q) ms.tl[q] = tl[q];
  }
  uint32_t theta = hist_bound(hist, ms.top_key, k);
  float xf = key_floor(theta ? theta : 1u);
  append_keys<kR0NV>(k0, 0, tid, theta ? theta : 1u, seg, cnt);
  if (mask) {   // (uniform)
    // The left-out ids after round 0 (the repetition set, or a deferring
    // row's listed ids) are streamed with their raw logits, which later
    // rounds may count: each is taken out of its bin first (before any wave
    // counts a later round).  Counted or not, the counts stay lower bounds of
    // the other logits' counts, and the raw entries are dropped at the end.
    const int e01 = 4 * round_base(1);
    auto take_out = [&](int id, float raw) {
      const uint32_t key = f2key(raw);
      if (id >= e01 && id < src.lim && key) atomicSub(&hist[key >> kMidShift], 1u);
    };
    if (pid >= 0) take_out(pid, pval);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int i = tid + c * kRowThreads;
      if (i < ne) take_out(eid[i], praw[c]);
    }
    __syncthreads();
  }

  // ---- rounds >= 1
  for (int r = 1; r < nr; r += 2) {
    mid_step(vb, round_base(r), tid, src.lim, k, hist, &ms.top_key, seg, cnt, theta, xf, lost);
    load_rd<kRowNV, VEC>(vb, src, round_base(r + 2), tid);   // past the row near its end
    if (r + 1 >= nr) break;
    mid_step(va, round_base(r + 1), tid, src.lim, k, hist, &ms.top_key, seg, cnt, theta, xf,
             lost);
    load_rd<kRowNV, VEC>(va, src, round_base(r + 3), tid);
  }
  lost = lost || cnt > kSegCap;

  // ---- end: penalised logits back in place (as in row_kernel)
  float pv = 0.f;
  if (pid >= 0) {
    RowPlan pr;
    pr.rep = load_scalar(&plan->rep);   // (read again: not held through the stream)
    pr.pen = kPenRep;
    pv = penalise(pval, true, 0u, pr);
    rowp[pid] = pv;
  }
  // a presence / frequency row's listed penalties (src/sampler.ts:24-33 and
  // the presence / frequency extension, as pen_kernel applies them), stored
  // in place; the fence makes the stores seen by a replay's reads
  if (ne > 0) {
    RowPlan pe{};   // (read again: not held through the stream)
    pe.pen = load_scalar(&plan->pen);
    pe.rep = load_scalar(&plan->rep);
    pe.pres = load_scalar(&plan->pres);
    pe.freq = load_scalar(&plan->freq);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int i = tid + c * kRowThreads;
      if (i < ne) {
        const uint32_t cw = eaux[i];
        const float v = penalise(praw[c], (cw >> 31) != 0, cw & 0x7FFFFFFFu, pe);
        eaux[i] = __float_as_uint(v);
        rowp[eid[i]] = v;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();   // every wave's counts are in
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  theta = hist_bound(hist, ms.top_key, k);
  const uint32_t lo = theta ? theta : 1u;
  xf = key_floor(lo);
  auto join = [&](bool pass, unsigned long long c) {
    const unsigned long long b = __ballot(pass);
    if (b) {
      const int leader = __ffsll((long long)b) - 1;
      int bp = 0;
      if (lane == leader) bp = atomicAdd(&ms.n_f, __popcll(b));
      bp = __shfl(bp, leader);
      const int p = bp + (int)lanes_below(b);
      if (pass && p < kSortCap) srt[p] = c;
    }
  };
  if (lost) {
    if (lane == 0) ms.ovf = 1;
  } else {
    // (the raw entries of left-out ids are dropped)
    for (int i = lane; i < cnt; i += 64) {
      const unsigned long long c = seg[i];
      const uint32_t id = cand_idx(c);
      join(cand_key(c) >= lo && !(mask && ((bitmap[id >> 5] >> (id & 31)) & 1u)), c);
    }
  }
  join(pid >= 0 && pv >= xf, pack_cand(f2key(pv), (uint32_t)pid));
  for (int i0 = 0; i0 < ne; i0 += kRowThreads) {   // (a presence / frequency row's listed ids)
    const int i = i0 + tid;
    const float ev = i < ne ? __uint_as_float(eaux[i]) : 0.f;
    join(i < ne && ev >= xf, pack_cand(f2key(ev), (uint32_t)(i < ne ? eid[i] : 0)));
  }
  if (VEC && src.lim < V) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int e = src.lim + q;
      const bool ok = tid == 0 && e < V && !(mask && ((bitmap[e >> 5] >> (e & 31)) & 1u));
      const float t = ms.tl[q];
      join(ok && t >= xf, pack_cand(f2key(t), (uint32_t)e));
    }
  }
  __syncthreads();
  const int n = ms.n_f;
  const bool overflow = ms.ovf != 0 || n > kSortCap;
  uint32_t T = 0;
  int n_sel = 0;
  if (!overflow) {
    // every entry's key is in [lo, top_key] (the penalised and tail logits
    // may exceed top_key: they share the top bin)
    sort_binned<kRowThreads>(srt, n, lo, ms.top_key, hist, cbuf);   // ends with a barrier
    if (n >= k) {
      // past the last entry equal to T (sorted: a binary search by every
      // thread, usually settled by the first read)
      T = cand_key(srt[k - 1]);
      int lo_i = k, hi_i = n;   // srt[lo_i - 1] == T; srt[hi_i] < T or hi_i == n
      if (k < n && cand_key(srt[k]) == T) {
        lo_i = k + 1;
        while (lo_i < hi_i) {
          const int mid = (lo_i + hi_i) >> 1;
          if (cand_key(srt[mid]) == T) lo_i = mid + 1; else hi_i = mid;
        }
      }
      n_sel = lo_i;
    } else {
      n_sel = n;
    }
  }
  RowPlan P;
  P.temperature = load_scalar(&plan->temperature);
  P.top_p = load_scalar(&plan->top_p);
  P.min_p = load_scalar(&plan->min_p);
  P.k = k;
  // the histogram's LDS becomes the tail's scratch
  RowScratch sc;
  sc.skey = hist;
  sc.sids = reinterpret_cast<int32_t *>(hist + kMaxK);
  sc.sprob = reinterpret_cast<float *>(hist + 2 * kMaxK);
  sc.sp = reinterpret_cast<double *>(hist + 3 * kMaxK);
  sc.rsv = reinterpret_cast<float *>(hist + 5 * kMaxK);
  sc.rsid = reinterpret_cast<int32_t *>(hist + 6 * kMaxK);
  // closed form: all finite logits are candidates and there are at most k
  finish_row<kRowThreads>(a, P, row, rowp, srt, n_sel, T, theta == 0 && n <= k, overflow, sc,
                          ms.tail);
}

// ---------------------------------------------------------------- chunk kernel

template <bool VEC>
__global__ __launch_bounds__(kThreads) void chunk_kernel(LaunchArgs a, Workspace ws) {
  __shared__ uint32_t repbits[kChunk / 32];
  __shared__ SelectSmem sel;
  __shared__ uint32_t s_thr[kWaves];
  __shared__ unsigned long long s_best[kWaves];
  __shared__ int32_t s_cnt, s_base, s_over;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = a.chunks;
  const int pos = blockIdx.x / S;
  const int chunk = blockIdx.x - pos * S;
  const int row = ws.chunk_list[pos];
  const RowPlan P = ws.plans[row];
  float *rowp = a.logits + (int64_t)row * a.stride;
  const int lo = chunk * kChunk;
  const int hi = min(lo + kChunk, a.vocab);
  const int wbase = lo + wave * kWaveSpan;

  // one HBM read of the chunk into registers (coalesced float4 per lane)
  float v[kNV][4];
#pragma unroll
  for (int j = 0; j < kNV; ++j) {
    const int e = wbase + (j * 64 + lane) * 4;
    if (VEC && e + 3 < hi) {
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(rowp + e));
      v[j][0] = t[0]; v[j][1] = t[1]; v[j][2] = t[2]; v[j][3] = t[3];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[j][q] = (e + q < hi) ? rowp[e + q] : __builtin_nanf("");
    }
  }

  // repetition penalty (rows without the extension; the pre-pass did those)
  if ((P.pen & kPenRep) && !(P.pen & kPenPF)) {
    for (int i = tid; i < kChunk / 32; i += kThreads) repbits[i] = 0;
    __syncthreads();
    const HistRow h = hist_row(a, row);
    const int64_t last = h.n < 128 ? h.n : 128;
    for (int64_t t = tid; t < last; t += kThreads) {
      const int id = h.p[hist_pos(h, h.n - last + t)];
      if (id >= lo && id < hi) atomicOr(&repbits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kNV; ++j) {
      const int e = wbase + (j * 64 + lane) * 4;
      if (e >= hi) continue;
      const int o = e - lo;
      const uint32_t bits = (repbits[o >> 5] >> (o & 31)) & 0xFu;
      if (bits) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (bits & (1u << q)) {
            const float nv = penalise(v[j][q], true, 0u, P);
            v[j][q] = nv;
            rowp[e + q] = nv;
          }
        }
      }
    }
  }

  ChunkInfo *info = ws.info + (int64_t)pos * S + chunk;
  uint2 *rowcand = ws.cand + (int64_t)pos * ((int64_t)S * kChunkCap);
  const int cap = S * kChunkCap;
  const int k = P.k;

  if (P.mode == kModeGreedy) {
    unsigned long long best = 0;
#pragma unroll
    for (int j = 0; j < kNV; ++j) {
      const int e = wbase + (j * 64 + lane) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t key = f2key(v[j][q]);
        const unsigned long long c = key ? pack_cand(key, (uint32_t)(e + q)) : 0ull;
        best = c > best ? c : best;
      }
    }
    best = wave_max64(best);
    if (lane == 0) s_best[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = s_best[0];
      for (int w = 1; w < kWaves; ++w) b = s_best[w] > b ? s_best[w] : b;
      info->best = b;
      info->thr = 0;
      info->finite = -1;
      info->overflow = 0;
    }
    return;
  }

  uint32_t X;
  int finite = -1;
  if (P.mode == kModeSmall) {
    // k-th largest lane maximum per wave: a lower bound of the chunk's k-th
    float lm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kNV; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) lm = fmaxf(lm, v[j][q]);
    const uint32_t mw = wave_kth_largest(f2key(lm), k);
    if (lane == 0) s_thr[wave] = mw;
    __syncthreads();
    X = max(max(s_thr[0], s_thr[1]), max(s_thr[2], s_thr[3]));
  } else {
    int total = 0;
    X = block_select<kThreads>(
        k,
        [&](int shift, uint32_t prefix, int pass) {
#pragma unroll
          for (int j = 0; j < kNV; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) hist_add(sel, f2key(v[j][q]), shift, prefix, pass);
        },
        sel, &total);
    finite = total;
  }
  if (X == 0) X = 1;   // fewer than k finite: keep every finite logit
  const float xf = key_floor(X);

  uint32_t mine = 0;
#pragma unroll
  for (int j = 0; j < kNV; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) mine += v[j][q] >= xf ? 1u : 0u;
  const uint32_t off = block_scan_incl<kThreads>(mine, sel.wsum) - mine;
  if (tid == kThreads - 1) s_cnt = (int)(off + mine);
  __syncthreads();
  if (tid == 0) {
    s_base = s_cnt ? atomicAdd(&ws.cand_count[pos], s_cnt) : 0;
    s_over = s_base + s_cnt > cap;
  }
  __syncthreads();
  int p = s_base + (int)off;
#pragma unroll
  for (int j = 0; j < kNV; ++j) {
    const int e = wbase + (j * 64 + lane) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (v[j][q] >= xf) {
        if (p < cap) rowcand[p] = make_uint2(f2key(v[j][q]), (uint32_t)(e + q));
        ++p;
      }
    }
  }
  if (tid == 0) {
    info->best = 0;
    info->thr = X;
    info->overflow = s_over;
    // with X == 1 every finite logit was kept, so the count is exact
    info->finite = (X == 1 && !s_over) ? s_cnt : finite;
  }
}

// ---------------------------------------------------------------- finalize

struct FinalSmem {
  SelectSmem sel;
  TailSmem tail;
  unsigned long long red[kWaves];
  uint32_t xrow;
  int32_t finite_sum, finite_known, overflow, n_all;
};

size_t finalize_smem_bytes() {
  return (size_t)kFinalCap * 8 + (size_t)kSortCap * 8 + (size_t)kMaxK * (4 + 4 + 4 + 8 + 4 + 4);
}

__global__ __launch_bounds__(kThreads) void finalize_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long fdyn[];
  unsigned long long *ent = fdyn;                    // kFinalCap
  unsigned long long *srt = fdyn + kFinalCap;        // kSortCap
  RowScratch s;
  s.sp = reinterpret_cast<double *>(srt + kSortCap); // kMaxK each below
  s.skey = reinterpret_cast<uint32_t *>(s.sp + kMaxK);
  s.sids = reinterpret_cast<int32_t *>(s.skey + kMaxK);
  s.sprob = reinterpret_cast<float *>(s.sids + kMaxK);
  s.rsv = s.sprob + kMaxK;
  s.rsid = reinterpret_cast<int32_t *>(s.rsv + kMaxK);
  __shared__ FinalSmem f;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = blockIdx.x;
  const int row = ws.chunk_list[pos];
  const int S = a.chunks;
  const RowPlan P = ws.plans[row];
  const float *rowp = a.logits + (int64_t)row * a.stride;
  const ChunkInfo *info = ws.info + (int64_t)pos * S;

  if (P.mode == kModeGreedy) {
    unsigned long long best = 0;
    for (int c = tid; c < S; c += kThreads) best = info[c].best > best ? info[c].best : best;
    best = wave_max64(best);
    if (lane == 0) f.red[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = f.red[0];
      for (int w = 1; w < kWaves; ++w) b = f.red[w] > b ? f.red[w] : b;
      write_greedy(a, row, rowp[0], b);
    }
    return;
  }

  const int k = P.k;
  if (tid == 0) {
    f.xrow = 0; f.finite_sum = 0; f.finite_known = 1; f.overflow = 0; f.n_all = 0;
  }
  __syncthreads();
  for (int c = tid; c < S; c += kThreads) {
    atomicMax(&f.xrow, info[c].thr);
    if (info[c].overflow) atomicOr(&f.overflow, 1);
    if (info[c].finite < 0) atomicAnd(&f.finite_known, 0);
    else atomicAdd(&f.finite_sum, info[c].finite);
  }
  __syncthreads();
  const int n_rowcand = min(ws.cand_count[pos], S * kChunkCap);
  const uint2 *rowcand = ws.cand + (int64_t)pos * ((int64_t)S * kChunkCap);
  const uint32_t xrow = f.xrow;
  const bool closed_form = f.finite_known && f.finite_sum <= k && !f.overflow;
  bool need_replay = f.overflow;

  // candidates >= X_row (a lower bound of the row's k-th largest) into LDS
  if (!need_replay) {
    for (int i = tid; i < n_rowcand; i += kThreads) {
      const uint2 c = rowcand[i];
      if (c.x >= xrow) {
        const int p = atomicAdd(&f.n_all, 1);
        if (p < kFinalCap) ent[p] = pack_cand(c.x, c.y);
      }
    }
    __syncthreads();
    if (f.n_all > kFinalCap) need_replay = true;
  }
  int n_sel = 0;
  uint32_t T = 0;
  if (!need_replay) {
    const int n_all = f.n_all;
    const SelResult sel = select_into<kThreads>(
        n_all, [ent](int p) { return ent[p]; }, 0u, k, srt, f.sel, f.tail);
    n_sel = sel.n_sel;
    T = sel.T;
    if (n_sel < 0) { need_replay = true; n_sel = 0; }
  }
  if (tid == 0) ws.cand_count[pos] = 0;   // ready for the next call
  finish_row<kThreads>(a, P, row, rowp, srt, n_sel, T, closed_form, need_replay, s, f.tail);
}

// ---------------------------------------------------------------- large-k kernel

// Rows with k > 1024 (up to topK = Infinity, src/sampler.ts:49): one
// 1024-thread workgroup per row making several passes over the row.
//   1. extremes: the packed maximum (value, lowest index), the smallest
//      finite key and n_F, the number of logits that can become candidates;
//   2. k < n_F only: T, the exact k-th largest key (12/12/8-bit radix
//      select).  The candidates are the logits above T plus k - #(> T) of
//      those equal to T.  With k >= n_F every such logit is a candidate and no
//      slot is ever evicted, so the reference's order is value descending,
//      index ascending (src/sampler.ts:50-73 with no replacement);
//   3. the normaliser S and a 4096-bucket histogram of candidate counts and
//      probability mass over the key range.  These binary64 sums run in
//      another order than the reference's (src/sampler.ts:82-86, 97, 108),
//      which moves probabilities by far less than the 1e-5 tolerance;
//   4. each position the tail needs (the top-p crossing, cutoff - 1, the
//      draw) is found from its bucket, narrowed by 1024-bucket passes until at
//      most 2048 logits remain, which are gathered into LDS, sorted and
//      walked in order.
// With k < n_F a group of equal values is ordered by slot history: when the
// drawn position falls in such a group the row reports HS_ROW_UNSUPPORTED
// and token -1 instead of guessing.

constexpr int kLT = 1024;      // threads per workgroup
constexpr int kLBins = 4096;   // level-1 buckets
constexpr int kLSub = 1024;    // refinement buckets
constexpr int kLCap = 2048;    // logits gathered and sorted in LDS
constexpr int kLWalk = 64;     // a bucket with more candidates is split once more

struct LargeSmem {
  uint32_t cnt[kLBins];
  double mass[kLBins];
  uint32_t cnt2[kLSub];
  double mass2[kLSub];
  unsigned long long buf[kLCap];
  double pbuf[kLCap];          // probability of buf[i] (binary64 of the f32 value)
  unsigned long long ured[kLT / 64];
  double dred[kLT / 64];
  // located bucket / element, published by one thread
  int32_t found, pos, id, tie, nbuf, hit;
  uint32_t key, b, ecnt;
  double emass, cum;
};

size_t large_smem_bytes() { return sizeof(LargeSmem); }

// Per-row constants of the large path (wave-uniform).
struct LargeRow {
  const float *rowp;
  int V, vec;
  uint32_t T;      // 0: every finite logit is a candidate; else keys > T plus `tin` equal to T
  int tin, teq;    // candidates equal to T, logits equal to T
  uint32_t lo, hi; // key range of the candidates
  int s1;          // level-1 bucket shift
  double m, inv_temp, S, inv_S;
};

__device__ __forceinline__ bool large_cand(const LargeRow &L, uint32_t key) {
  return key != 0u && key >= L.T;
}

// src/sampler.ts:83-89: probs[i] = f32(f32(exp((v - max) / T)) / S)
__device__ __forceinline__ float large_prob(const LargeRow &L, float v) {
  const double p = exp(((double)v - L.m) * L.inv_temp);
  return (float)((double)(float)p / L.S);
}

// exp(x) to about 1e-7 relative, for the passes over whole rows of the large
// path: x * log2(e) is split in binary64 into an integer n and r in
// [-1/2, 1/2]; 2^r comes from the hardware's binary32 exp2 and is scaled by
// 2^n.  Its results feed the normaliser and the positions (cumProb) of rows
// whose sums already run in another order than the reference's.
__device__ __forceinline__ double exp_fast(double x) {
  const double y = x * 1.4426950408889634074;   // log2(e)
  if (!(y > -2000.0)) return y != y ? y : 0.0;   // NaN stays NaN; far below: 0
  const double n = rint(y);
  const float r = (float)(y - n);
  return ldexp((double)__builtin_amdgcn_exp2f(r), (int)n);
}

// large_prob with exp_fast and a multiplication by 1/S: the probabilities
// the large path locates with.
__device__ __forceinline__ float large_pfast(const LargeRow &L, float v) {
  const double p = exp_fast(((double)v - L.m) * L.inv_temp);
  return (float)((double)(float)p * L.inv_S);
}

// Calls f(index, value) for every logit of the row.  Eight float4 (or, for
// unaligned rows, eight logits) per thread are requested before any is used,
// through a buffer resource: reads past the row return 0 and are skipped.
// The reads are cached (not non-temporal): the path makes several passes
// over a row, and the rows the GPU holds at once (607 KB each at V = 151936)
// fit the last-level cache, so the passes after the first are served there.
template <typename F>
__device__ __forceinline__ void large_pass(const LargeRow &L, F f) {
  constexpr int U = 8;
  const int tid = threadIdx.x;
  if (L.vec) {
    const int nfull = L.V >> 2;
    const rsrc_t r4 = make_rsrc(L.rowp, 16u * (uint32_t)nfull);
    for (int i0 = tid; i0 < nfull; i0 += U * kLT) {
      f32x4 t[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b128(r4, (i0 + u * kLT) * 16, 0, 0);
        t[u] = f32x4{__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                     __uint_as_float(x[3])};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kLT;
        if (i < nfull) {
          f(4 * i, t[u][0]); f(4 * i + 1, t[u][1]); f(4 * i + 2, t[u][2]); f(4 * i + 3, t[u][3]);
        }
      }
    }
    for (int e = 4 * nfull + tid; e < L.V; e += kLT) f(e, L.rowp[e]);
  } else {
    const rsrc_t r1 = make_rsrc(L.rowp, 4u * (uint32_t)L.V);
    for (int e0 = tid; e0 < L.V; e0 += U * kLT) {
      float t[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        t[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r1, (e0 + u * kLT) * 4, 0, 0));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * kLT;
        if (e < L.V) f(e, t[u]);
      }
    }
  }
}

__device__ __forceinline__ double wave_sum_f64(double x) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) x += __shfl_xor(x, m);
  return x;
}

__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long x, LargeSmem &sm) {
  x = wave_max64(x);
  if (lane_id() == 0) sm.ured[threadIdx.x >> 6] = x;
  __syncthreads();
  unsigned long long r = 0;
  for (int w = 0; w < kLT / 64; ++w) r = sm.ured[w] > r ? sm.ured[w] : r;
  __syncthreads();
  return r;
}

__device__ __forceinline__ unsigned long long block_sum_u64(unsigned long long x, LargeSmem &sm) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) x += __shfl_xor(x, m);
  if (lane_id() == 0) sm.ured[threadIdx.x >> 6] = x;
  __syncthreads();
  unsigned long long r = 0;
  for (int w = 0; w < kLT / 64; ++w) r += sm.ured[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ double block_sum_f64(double x, LargeSmem &sm) {
  x = wave_sum_f64(x);
  if (lane_id() == 0) sm.dred[threadIdx.x >> 6] = x;
  __syncthreads();
  double r = 0;
  for (int w = 0; w < kLT / 64; ++w) r += sm.dred[w];
  __syncthreads();
  return r;
}

// Exclusive prefix over the threads of the workgroup, in thread order, of a
// (count, mass) pair.
__device__ __forceinline__ void block_excl_scan2(uint32_t c, double m, uint32_t *ec, double *em,
                                                 LargeSmem &sm) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  uint32_t ic = c;
  double im = m;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t tc = __shfl_up(ic, d);
    const double tm = __shfl_up(im, d);
    if (lane >= d) { ic += tc; im += tm; }
  }
  if (lane == 63) { sm.ured[wave] = ic; sm.dred[wave] = im; }
  const uint32_t pc = __shfl_up(ic, 1);
  const double pm = __shfl_up(im, 1);
  __syncthreads();
  uint32_t bc = 0;
  double bm = 0;
  for (int w = 0; w < wave; ++w) { bc += (uint32_t)sm.ured[w]; bm += sm.dred[w]; }
  *ec = bc + (lane ? pc : 0u);
  *em = bm + (lane ? pm : 0.0);
  __syncthreads();
}

enum { kByMass = 0, kByPos = 1 };

// Whether a bucket holding positions [ec, ec + c) with mass [em, em + m)
// holds the located position.
__device__ __forceinline__ bool large_hit(int mode, double target, uint32_t pos, uint32_t ec,
                                          uint32_t c, double em, double m) {
  if (c == 0) return false;
  if (mode == kByPos) return ec <= pos && pos < ec + c;
  return em < target && em + m >= target;
}

// Located element of the candidate order.
struct LargeLoc {
  bool found;
  int pos, id;
  uint32_t key;
  bool tie;        // another candidate holds the same value
  double cum;      // cumProb through this position
};

// The id of the j-th logit (index order) whose key equals `key`.
__device__ __forceinline__ int large_nth_equal(const LargeRow &L, uint32_t key, uint32_t j, LargeSmem &sm) {
  const int tid = threadIdx.x;
  const int span = (L.V + kLT - 1) / kLT;
  const int b0 = tid * span, b1 = min(L.V, b0 + span);
  uint32_t c = 0;
  for (int e = b0; e < b1; ++e) c += f2key(L.rowp[e]) == key;
  uint32_t ec;
  double dummy;
  block_excl_scan2(c, 0.0, &ec, &dummy, sm);
  if (tid == 0) sm.id = -1;
  __syncthreads();
  if (ec <= j && j < ec + c) {
    uint32_t seen = ec;
    for (int e = b0; e < b1; ++e) {
      if (f2key(L.rowp[e]) == key) {
        if (seen == j) { sm.id = e; break; }
        ++seen;
      }
    }
  }
  __syncthreads();
  const int id = sm.id;
  __syncthreads();
  return id;
}

// Gathers the candidates with keys in [klo, khi] into sm.buf (sm.nbuf counts
// them, possibly past kLCap).  When more logits equal T than slots remain
// for them, which ones the reference keeps depends on its slot history: they
// are represented by `tin` placeholder entries (key T, id 0) instead.  With
// s2 >= 0 the same pass also fills the sub-histogram sm.cnt2 / sm.mass2 of
// the range by (key - klo) >> s2 (which must be cleared beforehand).
__device__ __forceinline__ void large_gather(const LargeRow &L, uint32_t klo, uint32_t khi, LargeSmem &sm,
                             int s2 = -1) {
  const bool btie = L.T != 0u && L.teq > L.tin;
  if (threadIdx.x == 0) sm.nbuf = 0;
  __syncthreads();
  // [klo, khi] as a value range (klo >= lo >= T, so its logits are all
  // candidates): two comparisons per logit, the key only for those inside.
  // The value range holds the key range (at most also +-0 when an end key is
  // the unused one below +0's), so the key is checked as well.
  const float flo = key_floor(klo), fhi = key2f(khi);
  large_pass(L, [&](int e, float v) {
    if (v >= flo && v <= fhi) {
      const uint32_t key = f2key(v);
      if (key < klo || key > khi) return;
      if (s2 >= 0) {
        const uint32_t b = (key - klo) >> s2;
        atomicAdd(&sm.cnt2[b], 1u);
        atomicAdd(&sm.mass2[b], (double)large_pfast(L, v));
      }
      if (!(btie && key == L.T)) {
        const int p = atomicAdd(&sm.nbuf, 1);
        if (p < kLCap) sm.buf[p] = pack_cand(key, (uint32_t)e);
      }
    }
  });
  __syncthreads();
  if (threadIdx.x == 0 && btie && L.T >= klo && L.T <= khi) {
    for (int i = 0; i < L.tin; ++i) {
      const int p = sm.nbuf++;
      if (p < kLCap) sm.buf[p] = pack_cand(L.T, 0u);
    }
  }
  __syncthreads();
}

// Finds the first position whose cumProb reaches `target` (kByMass) or the
// position `pos` (kByPos).  sm.cnt / sm.mass hold the level-1 histogram.
__device__ __forceinline__ LargeLoc large_locate(const LargeRow &L, int mode, double target, uint32_t pos,
                                 LargeSmem &sm) {
  const int tid = threadIdx.x;
  LargeLoc r;
  r.found = false; r.pos = -1; r.id = -1; r.key = 0; r.tie = false; r.cum = 0;
  // level 1: thread t owns buckets 4095-4t .. 4092-4t (descending values)
  {
    uint32_t c[4], tc = 0;
    double m[4], tm = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = kLBins - 1 - 4 * tid - i;
      c[i] = sm.cnt[b]; m[i] = sm.mass[b];
      tc += c[i]; tm += m[i];
    }
    uint32_t ec;
    double em;
    block_excl_scan2(tc, tm, &ec, &em, sm);
    if (tid == 0) sm.found = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (large_hit(mode, target, pos, ec, c[i], em, m[i])) {
        sm.found = 1; sm.b = (uint32_t)(kLBins - 1 - 4 * tid - i); sm.ecnt = ec; sm.emass = em;
      }
      ec += c[i]; em += m[i];
    }
    __syncthreads();
  }
  if (!sm.found) { __syncthreads(); return r; }
  uint32_t klo = L.lo + (sm.b << L.s1);
  uint32_t khi = (L.hi - klo) >> L.s1 ? klo + ((1u << L.s1) - 1u) : L.hi;
  uint32_t count = sm.cnt[sm.b];
  uint32_t Ec = sm.ecnt;
  double Em = sm.emass;
  __syncthreads();
  // narrow the bucket while it holds more logits than LDS sorts
  while (count > (uint32_t)kLCap && klo < khi) {
    int s2 = 0;
    while (((khi - klo) >> s2) >= (uint32_t)kLSub) ++s2;
    sm.cnt2[tid] = 0;
    sm.mass2[tid] = 0;
    __syncthreads();
    const float flo = key_floor(klo), fhi = key2f(khi);   // as in large_gather
    large_pass(L, [&](int, float v) {
      if (v >= flo && v <= fhi) {
        const uint32_t key = f2key(v);
        if (key < klo || key > khi) return;
        const uint32_t b = (key - klo) >> s2;
        atomicAdd(&sm.cnt2[b], 1u);
        atomicAdd(&sm.mass2[b], (double)large_pfast(L, v));
      }
    });
    __syncthreads();
    if (tid == 0 && L.T && L.teq > L.tin && L.T >= klo && L.T <= khi) {
      const uint32_t b = (L.T - klo) >> s2;   // only `tin` of the T-valued logits count
      sm.cnt2[b] -= (uint32_t)(L.teq - L.tin);
      sm.mass2[b] -= (double)(L.teq - L.tin) * (double)large_pfast(L, key2f(L.T));
    }
    __syncthreads();
    const int b = kLSub - 1 - tid;
    const uint32_t c = sm.cnt2[b];
    const double m = sm.mass2[b];
    uint32_t ec;
    double em;
    block_excl_scan2(c, m, &ec, &em, sm);
    ec += Ec; em += Em;
    if (tid == 0) sm.found = 0;
    __syncthreads();
    if (large_hit(mode, target, pos, ec, c, em, m)) {
      sm.found = 1; sm.b = (uint32_t)b; sm.ecnt = ec; sm.emass = em;
    }
    __syncthreads();
    if (!sm.found) { __syncthreads(); return r; }
    const uint32_t nlo = klo + (sm.b << s2);
    khi = (khi - nlo) >> s2 ? nlo + ((1u << s2) - 1u) : khi;
    klo = nlo;
    count = sm.cnt2[sm.b];
    Ec = sm.ecnt;
    Em = sm.emass;
    __syncthreads();
  }
  if (count > (uint32_t)kLCap) {
    // one value held by more logits than LDS sorts: equal probabilities,
    // index order (the reference's order when no slot was evicted)
    const uint32_t key = klo;
    const float pv = large_pfast(L, key2f(key));
    uint32_t j = 0;
    double c = Em;
    if (mode == kByPos) {
      j = pos - Ec;
      for (uint32_t i = 0; i <= j; ++i) c += (double)pv;
    } else {
      for (j = 0; j < count; ++j) {
        c += (double)pv;
        if (c >= target) break;
      }
      if (j == count) { j = count - 1; }
    }
    r.found = true; r.pos = (int)(Ec + j); r.key = key; r.tie = true; r.cum = c;
    r.id = large_nth_equal(L, key, j, sm);
    return r;
  }
  // Gather the bucket's logits.  When it spans several keys and holds more
  // than kLWalk candidates, the same pass builds its sub-histogram; only the
  // sub-bucket holding the position is then kept, sorted and walked.
  if (count > (uint32_t)kLWalk && klo < khi) {
    int s2 = 0;
    while (((khi - klo) >> s2) >= (uint32_t)kLSub) ++s2;
    sm.cnt2[tid] = 0;
    sm.mass2[tid] = 0;
    __syncthreads();
    large_gather(L, klo, khi, sm, s2);
    if (tid == 0 && L.T && L.teq > L.tin && L.T >= klo && L.T <= khi) {
      const uint32_t b = (L.T - klo) >> s2;   // only `tin` of the T-valued logits count
      sm.cnt2[b] -= (uint32_t)(L.teq - L.tin);
      sm.mass2[b] -= (double)(L.teq - L.tin) * (double)large_pfast(L, key2f(L.T));
    }
    __syncthreads();
    const int b = kLSub - 1 - tid;
    const uint32_t c = sm.cnt2[b];
    const double m = sm.mass2[b];
    uint32_t ec;
    double em;
    block_excl_scan2(c, m, &ec, &em, sm);
    ec += Ec; em += Em;
    if (tid == 0) sm.found = 0;
    __syncthreads();
    if (large_hit(mode, target, pos, ec, c, em, m)) {
      sm.found = 1; sm.b = (uint32_t)b; sm.ecnt = ec; sm.emass = em;
    }
    __syncthreads();
    if (sm.found) {   // else: rounding at the bucket's edge, walk it whole
      const uint32_t nlo = klo + (sm.b << s2);
      khi = (khi - nlo) >> s2 ? nlo + ((1u << s2) - 1u) : khi;
      klo = nlo;
      count = sm.cnt2[sm.b];
      Ec = sm.ecnt;
      Em = sm.emass;
      // keep the gathered entries of the sub-bucket (through pbuf's storage)
      unsigned long long *tmp = reinterpret_cast<unsigned long long *>(sm.pbuf);
      const int nall = min(sm.nbuf, kLCap);
      __syncthreads();
      if (tid == 0) sm.hit = 0;
      __syncthreads();
      for (int i = tid; i < nall; i += kLT) {
        const unsigned long long e = sm.buf[i];
        const uint32_t key = cand_key(e);
        if (key >= klo && key <= khi) tmp[atomicAdd(&sm.hit, 1)] = e;
      }
      __syncthreads();
      const int nk = sm.hit;
      for (int i = tid; i < nk; i += kLT) sm.buf[i] = tmp[i];
      if (tid == 0) sm.nbuf = nk;
      __syncthreads();
    }
  } else {
    large_gather(L, klo, khi, sm);
  }
  const int nb = min(sm.nbuf, kLCap);
  sort_packed<kLT>(sm.buf, nb);
  // T-valued logits past `tin` are not candidates (the list holds at most tin)
  const int nv = nb < (int)count ? nb : (int)count;
  if (tid == 0) sm.hit = nv;
  int bad = 0;
  for (int i = tid; i < nv; i += kLT) {
    const float pf = large_pfast(L, key2f(cand_key(sm.buf[i])));
    sm.pbuf[i] = (double)pf;
    bad |= !((double)pf == 0.0 || ((double)pf >= 0x1p-29 && (double)pf <= 1.0));
  }
  if (!__syncthreads_or(bad)) {
    // Every probability is a multiple of 2^-52: the prefix sums are exact in
    // any order (see wave_tail), so the walk is a block prefix sum; pbuf[i]
    // becomes cumProb through position Ec + i.
    const int lane = tid & 63, wave = tid >> 6;
    double carry = Em;
    for (int base = 0; base < nv; base += kLT) {
      const int i = base + tid;
      double c = wave_scan_incl_f64(i < nv ? sm.pbuf[i] : 0.0);
      __syncthreads();
      if (lane == 63) sm.dred[wave] = c;
      __syncthreads();
      double add = carry, tot = carry;
      for (int w = 0; w < kLT / 64; ++w) {
        if (w < wave) add += sm.dred[w];
        tot += sm.dred[w];
      }
      c += add;
      if (i < nv) {
        sm.pbuf[i] = c;
        if (mode == kByPos ? Ec + (uint32_t)i == pos : c >= target) atomicMin(&sm.hit, i);
      }
      carry = tot;
    }
    __syncthreads();
    if (tid == 0) {
      const int hit = sm.hit < nv ? sm.hit : (nv > 0 ? nv - 1 : 0);   // past the end: its last logit
      const uint32_t key = cand_key(sm.buf[hit]);
      sm.pos = (int)Ec + hit;
      sm.id = (int)cand_idx(sm.buf[hit]);
      sm.key = key;
      sm.cum = nv > 0 ? sm.pbuf[hit] : Em;
      sm.tie = (hit > 0 && cand_key(sm.buf[hit - 1]) == key) ||
               (hit + 1 < nb && cand_key(sm.buf[hit + 1]) == key);
    }
  } else if (tid == 0) {
    double c = Em;
    int hit = -1, tseen = 0;
    const int avail = (int)count;   // T-valued logits past `tin` are not candidates
    int j = 0;
    for (; j < nb && j < avail; ++j) {
      const uint32_t key = cand_key(sm.buf[j]);
      if (L.T && key == L.T && tseen++ >= L.tin) break;
      c += sm.pbuf[j];
      if (mode == kByPos ? Ec + (uint32_t)j == pos : c >= target) { hit = j; break; }
    }
    if (hit < 0) { hit = j > 0 ? j - 1 : 0; }   // rounding at a bucket edge: its last logit
    const uint32_t key = cand_key(sm.buf[hit]);
    sm.pos = (int)Ec + hit;
    sm.id = (int)cand_idx(sm.buf[hit]);
    sm.key = key;
    sm.cum = c;
    sm.tie = (hit > 0 && cand_key(sm.buf[hit - 1]) == key) ||
             (hit + 1 < nb && cand_key(sm.buf[hit + 1]) == key);
  }
  __syncthreads();
  r.found = true; r.pos = sm.pos; r.id = sm.id; r.key = sm.key; r.tie = sm.tie != 0; r.cum = sm.cum;
  __syncthreads();
  return r;
}

// The general large-k path for one row: any k > 1024, min-p, candidate
// outputs, and the rows the two-pass path below hands back.
// With k below the finite count, an equal-value group whose order decides
// the token or the candidate list is left to a slot replay through *req:
// large_replay_kernel (slots in LDS) for k <= kReplayMaxK and at most
// kReplayCands candidate positions, large_replay_dev_kernel (slots in device
// memory) up to k = kReplayDevMaxK and kReplayDevCands positions; beyond
// those the row reports HS_ROW_UNSUPPORTED.
__device__ __forceinline__ void large_row(const LaunchArgs &a, const RowPlan &P, int row,
                                          LargeSmem &sm, ReplayReq *req) {
  const int tid = threadIdx.x;
  if (tid == 0) req->need = 0;
  LargeRow L;
  L.rowp = a.logits + (int64_t)row * a.stride;
  L.V = a.vocab;
  L.vec = a.vec;
  L.T = 1u;       // every finite logit, for the first passes
  L.tin = L.teq = 0;

  // 1. extremes and n_F.  A thread meets its logits in index order, so its
  // first maximum is kept by the strict comparison.
  uint32_t bkey = 0, bidx = 0, kmin = 0xFFFFFFFFu, nf = 0;
  large_pass(L, [&](int e, float v) {
    const uint32_t key = f2key(v);
    const bool gt = key > bkey;
    bkey = gt ? key : bkey;
    bidx = gt ? (uint32_t)e : bidx;
    const uint32_t km = key ? key : 0xFFFFFFFFu;
    kmin = km < kmin ? km : kmin;
    nf += key != 0u;
  });
  const unsigned long long best = block_max_u64(bkey ? pack_cand(bkey, bidx) : 0ull, sm);
  const uint32_t kmin_all = ~(uint32_t)block_max_u64((unsigned long long)(~kmin), sm);
  const int n_f = (int)block_sum_u64(nf, sm);
  const int k = P.k;
  const int n = k < n_f ? k : n_f;
  const int cs = a.cand_stride;

  if (n <= 1) {   // src/sampler.ts:76-77: no draw
    if (tid == 0) {
      put_token(a, row, n == 1 ? (int)cand_idx(best) : 0);
      if (a.cand_count_out) a.cand_count_out[row] = n;
      if (a.cutoff_out) a.cutoff_out[row] = n;
      if (a.row_flags) a.row_flags[row] = HS_ROW_SINGLE | HS_ROW_LARGE;
      if (n == 1 && cs > 0) {
        if (a.cand_ids) a.cand_ids[(int64_t)row * cs] = (int)cand_idx(best);
        if (a.cand_probs) a.cand_probs[(int64_t)row * cs] = 1.0f;
      }
    }
    return;
  }

  // 2. k < n_F: T = the exact k-th largest key
  L.T = 0u;
  if (k < n_f) {
    uint32_t prefix = 0;
    int rem = k;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = pass == 0 ? 20 : (pass == 1 ? 8 : 0);
      const int nbits = pass == 2 ? 8 : 12;
      const int nb = 1 << nbits, top = sh + nbits;
      for (int i = tid; i < kLBins; i += kLT) sm.cnt[i] = 0;
      __syncthreads();
      large_pass(L, [&](int, float v) {
        const uint32_t key = f2key(v);
        if (key && (pass == 0 || (key >> top) == (prefix >> top)))
          atomicAdd(&sm.cnt[(key >> sh) & (uint32_t)(nb - 1)], 1u);
      });
      __syncthreads();
      // thread t owns digits nb-1-4t .. nb-4-4t (descending)
      uint32_t c[4], tc = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = nb - 1 - 4 * tid - i;
        c[i] = d >= 0 ? sm.cnt[d] : 0u;
        tc += c[i];
      }
      uint32_t ec;
      double dummy;
      block_excl_scan2(tc, 0.0, &ec, &dummy, sm);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (ec < (uint32_t)rem && ec + c[i] >= (uint32_t)rem) {
          sm.b = (uint32_t)(nb - 1 - 4 * tid - i);
          sm.ecnt = ec;
          sm.nbuf = (int)c[i];
        }
        ec += c[i];
      }
      __syncthreads();
      prefix |= sm.b << sh;
      rem -= (int)sm.ecnt;
      L.teq = sm.nbuf;
      __syncthreads();
    }
    L.T = prefix;
    L.tin = rem;            // k - #(> T) slots left for the T-valued logits
  }
  L.lo = L.T ? L.T : kmin_all;
  L.hi = cand_key(best);
  L.s1 = 0;
  while (((L.hi - L.lo) >> L.s1) >= (uint32_t)kLBins) ++L.s1;
  L.m = (double)key2f(L.hi);
  L.inv_temp = 1.0 / P.temperature;

  // 3. normaliser and level-1 histogram in one pass.  A bucket sums the
  // binary32-rounded exp values and is divided by S afterwards: its mass then
  // differs from the sum of its binary32 probabilities by their rounding only.
  for (int i = tid; i < kLBins; i += kLT) { sm.cnt[i] = 0; sm.mass[i] = 0; }
  __syncthreads();
  double s = 0;
  large_pass(L, [&](int, float v) {
    const uint32_t key = f2key(v);
    if (key != 0u && key > L.T) {
      const double p = exp_fast(((double)v - L.m) * L.inv_temp);
      s += p;
      const uint32_t b = (key - L.lo) >> L.s1;
      atomicAdd(&sm.cnt[b], 1u);
      atomicAdd(&sm.mass[b], (double)(float)p);
    }
  });
  const double pT = L.T ? exp_fast(((double)key2f(L.T) - L.m) * L.inv_temp) : 0.0;
  L.S = block_sum_f64(s, sm) + (double)L.tin * pT;   // ends with a barrier
  L.inv_S = 1.0 / L.S;
  if (tid == 0 && L.T) {
    sm.cnt[0] += (uint32_t)L.tin;   // T is the lowest candidate key: bucket 0
    sm.mass[0] += (double)L.tin * (double)(float)pT;
  }
  __syncthreads();
  for (int i = tid; i < kLBins; i += kLT) sm.mass[i] *= L.inv_S;
  const float prob0 = large_pfast(L, key2f(L.hi));
  const double thr = P.min_p * (double)prob0;
  // candidates with !(prob < thr) (src/sampler.ts:96): all of them unless
  // thr > 0, which needs one more pass
  unsigned long long nlt = (unsigned long long)n;
  if (thr > 0.0) {
    nlt = 0;
    large_pass(L, [&](int, float v) {
      const uint32_t key = f2key(v);
      if (key != 0u && key > L.T) nlt += !((double)large_pfast(L, v) < thr);
    });
    nlt = block_sum_u64(nlt, sm);
    if (L.T) nlt += !((double)large_pfast(L, key2f(L.T)) < thr) ? (unsigned long long)L.tin : 0ull;
  }
  __syncthreads();

  // 4. src/sampler.ts:93-105: min-p stop f1, top-p stop f2
  int f1 = 1 + (int)nlt - (!((double)prob0 < thr) ? 1 : 0);
  f1 = f1 < 1 ? 1 : (f1 > n ? n : f1);
  int f2 = n;
  LargeLoc f2_loc;
  f2_loc.found = false;
  if (P.top_p <= 0.0) {
    f2 = 0;   // cumProb >= topP at the first index
  } else {
    f2_loc = large_locate(L, kByMass, P.top_p, 0u, sm);
    if (f2_loc.found) f2 = f2_loc.pos;
  }
  int cut = f1 <= f2 ? f1 : f2 + 1;
  cut = cut > n ? n : cut;
  // src/sampler.ts:107-116: keptSum = cumProb at cutoff - 1 (the top-p
  // position itself when the top-p stop sets the cutoff), then the draw
  const LargeLoc lkept = cut == f2 + 1 && f2_loc.found
                             ? f2_loc
                             : large_locate(L, kByPos, 0.0, (uint32_t)(cut - 1), sm);
  const double target = a.uniforms[row] * lkept.cum;
  LargeLoc lpick = large_locate(L, kByMass, target, 0u, sm);
  if (!lpick.found || lpick.pos >= cut) lpick = lkept;
  if (!(target > 0.0) && target == target) {
    // r = u * keptSum <= 0: the first subtraction already ends the walk
    lpick = large_locate(L, kByPos, 0.0, 0u, sm);
  }
  const bool ambiguous = L.T != 0u && lpick.tie;   // slot history orders equal values
  const bool replay = ambiguous && k <= kReplayDevMaxK;
  uint32_t flags = HS_ROW_LARGE;
  if (ambiguous) flags |= HS_ROW_TIES | (replay ? HS_ROW_REPLAYED : HS_ROW_UNSUPPORTED);
  int need = replay ? 1 : 0, need_mo = 0;
  uint32_t need_ckey = 0;
  if (tid == 0) {
    if (!replay) put_token(a, row, ambiguous ? -1 : lpick.id);
    if (a.cand_count_out) a.cand_count_out[row] = n;
    if (a.cutoff_out) a.cutoff_out[row] = cut;
  }

  // candidate outputs: the first min(n, cand_stride) positions.  The values
  // above the last position's value are gathered and sorted; the last value's
  // group fills the rest in index order.
  if (cs > 0 && (a.cand_ids || a.cand_probs)) {
    const int mo = n < cs ? n : cs;
    const LargeLoc lend = large_locate(L, kByPos, 0.0, (uint32_t)(mo - 1), sm);
    const uint32_t kend = lend.key;
    large_gather(L, kend + 1u, L.hi, sm);   // kend < hi or nothing lies above
    int nb = kend < L.hi ? sm.nbuf : 0;     // < mo: they precede position mo - 1
    const bool too_long = nb > kLCap;       // a list longer than LDS sorts
    if (too_long) {
      flags |= HS_ROW_UNSUPPORTED;
      nb = 0;
    }
    int P2 = 1;
    while (P2 < nb) P2 <<= 1;
    for (int i = nb + tid; i < P2; i += kLT) sm.buf[i] = 0ull;
    __syncthreads();
    block_sort_desc<kLT>(sm.buf, P2);
    int tie = 0;
    for (int i = tid; i < nb; i += kLT) {
      const unsigned long long c = sm.buf[i];
      if (a.cand_ids) a.cand_ids[(int64_t)row * cs + i] = (int32_t)cand_idx(c);
      if (a.cand_probs) a.cand_probs[(int64_t)row * cs + i] = large_prob(L, key2f(cand_key(c)));
      if (i + 1 < nb && cand_key(sm.buf[i + 1]) == cand_key(c)) tie = 1;
    }
    // the group of the last listed value, in index order
    const int rest = mo - nb;
    const float pend = large_prob(L, key2f(kend));
    const int span = (L.V + kLT - 1) / kLT;
    const int b0 = tid * span, b1 = min(L.V, b0 + span);
    uint32_t c = 0;
    if (!too_long)
      for (int e = b0; e < b1; ++e) c += f2key(L.rowp[e]) == kend;
    uint32_t ec;
    double dummy;
    block_excl_scan2(c, 0.0, &ec, &dummy, sm);
    for (int e = b0; e < b1 && ec < (uint32_t)rest; ++e) {
      if (f2key(L.rowp[e]) == kend) {
        const int i = nb + (int)ec++;
        if (a.cand_ids) a.cand_ids[(int64_t)row * cs + i] = e;
        if (a.cand_probs) a.cand_probs[(int64_t)row * cs + i] = pend;
      }
    }
    if (rest > 1 || (kend == L.T && L.teq > L.tin)) tie = 1;
    if (__syncthreads_or(tie) && L.T) {
      if (k <= kReplayDevMaxK && mo <= kReplayDevCands && !too_long) {
        need |= 2;
        need_mo = mo;
        need_ckey = kend;
        flags |= HS_ROW_TIES | HS_ROW_REPLAYED;
      } else {
        flags |= HS_ROW_UNSUPPORTED | HS_ROW_TIES;
      }
    }
  }
  // slots beyond the LDS replay's, or more positions than it orders: the
  // device-memory replay
  if (need && (k > kReplayMaxK || need_mo > kReplayCands)) need |= kReplayDev;
  if (tid == 0) {
    if (a.row_flags) a.row_flags[row] = flags;
    req->xkey = lpick.key;
    req->pos = lpick.pos;
    req->mo = need_mo;
    req->ckey = need_ckey;
    req->need = need;
  }
}

// ---------------------------------------------------------------- large-k slot replay

// src/sampler.ts:50-69 replayed for a row whose equal values large_row could
// not order (k <= kReplayMaxK, below the finite count).  The k slots live in
// LDS under a 64-ary min tree: lvl1[b] is the smallest (key, slot) of slots
// 64b .. 64b+63, lvl2[c] of lvl1 entries 64c .. 64c+63, and the root of
// lvl2 is the slot the reference's rescan finds (the first slot holding the
// minimum: packed (key << 32 | slot), an empty slot's key 0).
//  - The first k finite logits fill slots 0..k-1 in index order (the rescan
//    always finds the first empty slot), placed in parallel.
//  - Then the row is read in chunks of kLT logits; those above the chunk's
//    starting minimum queue up in index order, and one wave takes them one
//    by one: a logit above the current minimum replaces that slot, and the
//    three tree levels on its path are recomputed (a 64-lane minimum each).
//  - The final slots then order each equal-value group by slot index (the
//    stable sort of src/sampler.ts:72-75): the token is the member of the
//    drawn value at the drawn rank, and the candidate ids follow
//    (value descending, slot ascending).
struct ReplaySmem {
  uint32_t keys[kReplayMaxK];
  int32_t ids[kReplayMaxK];
  unsigned long long lvl1[kReplayMaxK / 64];
  unsigned long long lvl2[kReplayMaxK / 4096];
  unsigned long long queue[kLT];
  uint32_t wsum[kLT / 64];
  int32_t nq, fill_end, res;
  unsigned long long root;
};
size_t replay_smem_bytes() { return sizeof(ReplaySmem); }

__device__ __forceinline__ unsigned long long wave_min64(unsigned long long x) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const unsigned long long y = __shfl_xor(x, m);
    x = x < y ? x : y;
  }
  return x;
}

__device__ __forceinline__ unsigned long long slot_pack(uint32_t key, uint32_t slot) {
  return ((unsigned long long)key << 32) | slot;
}

__global__ __launch_bounds__(kLT) void large_replay_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long rdyn[];
  ReplaySmem &sm = *reinterpret_cast<ReplaySmem *>(rdyn);
  const ReplayReq req = ws.large_replay[blockIdx.x];
  if (!req.need || (req.need & kReplayDev)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = ws.large_list[blockIdx.x];
  const int k = ws.plans[row].k;
  const float *rowp = a.logits + (int64_t)row * a.stride;
  const int V = a.vocab;
  constexpr unsigned long long kNone = ~0ull;
  // inclusive block prefix of x, and the block's total
  auto scan = [&](uint32_t x, uint32_t &total) {
    const uint32_t incl = block_scan_incl<kLT>(x, sm.wsum);
    uint32_t t = 0;
    for (int w = 0; w < kLT / 64; ++w) t += sm.wsum[w];
    total = t;
    __syncthreads();   // before wsum is used again
    return incl;
  };

  // 1. the first k finite logits fill slots 0..k-1 in index order
  if (tid == 0) sm.fill_end = V;
  int filled = 0;
  for (int base = 0; base < V && filled < k; base += kLT) {
    const int e = base + tid;
    const uint32_t key = e < V ? f2key(rowp[e]) : 0u;
    uint32_t total;
    const uint32_t incl = scan(key ? 1u : 0u, total);
    const int slot = filled + (int)incl - 1;
    if (key && slot < k) {
      sm.keys[slot] = key;
      sm.ids[slot] = e;
      if (slot == k - 1) sm.fill_end = e + 1;
    }
    filled += (int)total;
  }
  for (int s = filled + tid; s < k; s += kLT) { sm.keys[s] = 0u; sm.ids[s] = -1; }
  __syncthreads();
  const int nl1 = (k + 63) >> 6, nl2 = (nl1 + 63) >> 6;
  for (int b = wave; b < nl1; b += kLT / 64) {
    const int sl = 64 * b + lane;
    const unsigned long long m = wave_min64(sl < k ? slot_pack(sm.keys[sl], (uint32_t)sl) : kNone);
    if (lane == 0) sm.lvl1[b] = m;
  }
  __syncthreads();
  if (wave == 0) {
    unsigned long long top = kNone;
    for (int c = 0; c < nl2; ++c) {
      const int i = 64 * c + lane;
      const unsigned long long m = wave_min64(i < nl1 ? sm.lvl1[i] : kNone);
      if (lane == 0) sm.lvl2[c] = m;
      top = m < top ? m : top;
    }
    if (lane == 0) sm.root = top;
  }
  __syncthreads();

  // 2. the rest of the row, in index order
  const int start = sm.fill_end;
  for (int base = start; base < V; base += kLT) {
    const uint32_t lo = (uint32_t)(sm.root >> 32);   // the minimum at the chunk's start
    const int e = base + tid;
    const uint32_t key = e < V ? f2key(rowp[e]) : 0u;
    const bool enter = key > lo;
    uint32_t total;
    const uint32_t incl = scan(enter ? 1u : 0u, total);
    if (enter) sm.queue[incl - 1] = slot_pack(key, (uint32_t)e);
    const int nq = (int)total;
    __syncthreads();
    if (wave == 0) {
      unsigned long long top = sm.root;
      for (int q = 0; q < nq; ++q) {
        const unsigned long long item = sm.queue[q];
        const uint32_t kv = (uint32_t)(item >> 32);
        if (kv <= (uint32_t)(top >> 32)) continue;   // not above the current minimum
        const int s = (int)(uint32_t)top;
        if (lane == 0) {
          sm.keys[s] = kv;
          sm.ids[s] = (int)(uint32_t)item;
        }
        const int b1 = s >> 6, sl = 64 * b1 + lane;
        const unsigned long long m1 = wave_min64(
            sl < k ? slot_pack(sl == s ? kv : sm.keys[sl], (uint32_t)sl) : kNone);
        const int b2 = b1 >> 6, i1 = 64 * b2 + lane;
        const unsigned long long m2 = wave_min64(i1 < nl1 ? (i1 == b1 ? m1 : sm.lvl1[i1]) : kNone);
        const unsigned long long m3 = wave_min64(lane < nl2 ? (lane == b2 ? m2 : sm.lvl2[lane]) : kNone);
        if (lane == 0) {
          sm.lvl1[b1] = m1;
          sm.lvl2[b2] = m2;
        }
        top = m3;
      }
      if (lane == 0) sm.root = top;
    }
    __syncthreads();
  }

  // 3. the token: the member of the drawn value at its rank in slot order
  const int span = (k + kLT - 1) / kLT;
  const int s0 = tid * span, s1 = min(k, s0 + span);
  if (req.need & 1) {
    uint32_t above = 0, eq = 0;
    for (int s = s0; s < s1; ++s) {
      above += sm.keys[s] > req.xkey;
      eq += sm.keys[s] == req.xkey;
    }
    uint32_t n_above, n_eq;
    (void)scan(above, n_above);
    const uint32_t incl = scan(eq, n_eq);
    const int j = req.pos - (int)n_above;     // rank in the group
    if (tid == 0) sm.res = -1;
    __syncthreads();
    uint32_t seen = incl - eq;
    if (j >= 0 && (uint32_t)j >= seen && (uint32_t)j < incl) {
      for (int s = s0; s < s1; ++s) {
        if (sm.keys[s] == req.xkey) {
          if (seen == (uint32_t)j) { sm.res = sm.ids[s]; break; }
          ++seen;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      put_token(a, row, sm.res);
      if (sm.res < 0 && a.row_flags) a.row_flags[row] |= HS_ROW_UNSUPPORTED;
    }
    __syncthreads();
  }

  // 4. the candidate ids of positions 0..mo-1 (value descending, slot
  // ascending): the mo largest (key << 32 | ~slot), by a search for the key
  // at position mo - 1 and a sort of at most mo entries
  if ((req.need & 2) && a.cand_ids) {
    const int mo = req.mo;
    uint32_t lo = 1, hi = 0xFFFFFFFFu;   // largest key t with count(key >= t) >= mo
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo + 1) / 2;
      uint32_t c = 0, tot;
      for (int s = s0; s < s1; ++s) c += sm.keys[s] >= mid;
      (void)scan(c, tot);
      if (tot >= (uint32_t)mo) lo = mid; else hi = mid - 1;
    }
    const uint32_t X = lo;
    uint32_t gt = 0, eq = 0;
    for (int s = s0; s < s1; ++s) {
      gt += sm.keys[s] > X;
      eq += sm.keys[s] == X;
    }
    uint32_t n_gt, n_eq;
    const uint32_t ig = scan(gt, n_gt);
    const uint32_t ie = scan(eq, n_eq);
    uint32_t pg = ig - gt, pe = ie - eq;
    for (int s = s0; s < s1; ++s) {
      const uint32_t key = sm.keys[s];
      if (key > X) sm.queue[pg++] = pack_cand(key, (uint32_t)s);
      else if (key == X && n_gt + pe < (uint32_t)mo) sm.queue[n_gt + pe++] = pack_cand(key, (uint32_t)s);
      else if (key == X) ++pe;
    }
    __syncthreads();
    int P2 = 1;
    while (P2 < mo) P2 <<= 1;
    for (int i = mo + tid; i < P2; i += kLT) sm.queue[i] = 0ull;
    __syncthreads();
    block_sort_desc<kLT>(sm.queue, P2);
    const int cs = a.cand_stride;
    for (int i = tid; i < mo; i += kLT)
      a.cand_ids[(int64_t)row * cs + i] = sm.ids[cand_idx(sm.queue[i])];
  }
}

// ---------------------------------------------------------------- large-k slot replay, slots in device memory

// The same replay of src/sampler.ts:50-69 for the rows whose k slots do not
// fit in LDS (k > kReplayMaxK, up to kReplayDevMaxK), or whose candidate
// outputs need more ordered positions than the LDS replay takes.  The slots'
// keys and ids, and the first level of the min tree above them (lvl1, the
// minimum of each 64 slots), live in the workgroup's region of the
// workspace; lvl2 (over 64 lvl1 entries) and lvl3 (over 64 lvl2 entries,
// at most 64 of them) stay in LDS, and the root is the minimum of lvl3.
// The lane that writes a slot or a lvl1 entry is the lane that reads it
// back (its index & 63), so every read of one written during the replay is
// ordered after that write by the thread's own program order.  The grid
// holds at most kReplayDevBlocks workgroups, each taking
// the requesting rows whose rank among them is its index modulo the grid,
// one after the other: the workspace needs one region per workgroup, not
// one per row.
struct ReplayDevSmem {
  unsigned long long lvl2[kReplayDevMaxK / 4096];
  unsigned long long lvl3[64];
  unsigned long long buf[kReplayDevCands];   // the chunk's entering logits, then the sort
  int32_t rows[kLT];                         // this workgroup's rows of a list chunk
  uint32_t wsum[kLT / 64];
  int32_t fill_end, res;
  unsigned long long root;
};
size_t replay_dev_smem_bytes() { return sizeof(ReplayDevSmem); }
static_assert(kReplayDevMaxK <= 64 * 64 * 64 * 64, "lvl3 holds at most 64 entries");

__device__ void replay_dev_row(const LaunchArgs &a, const Workspace &ws, const ReplayReq &req,
                               int row, uint32_t *keys, int32_t *ids,
                               unsigned long long *lvl1, ReplayDevSmem &sm) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int k = ws.plans[row].k;
  const float *rowp = a.logits + (int64_t)row * a.stride;
  const int V = a.vocab;
  constexpr unsigned long long kNone = ~0ull;
  auto scan = [&](uint32_t x, uint32_t &total) {
    const uint32_t incl = block_scan_incl<kLT>(x, sm.wsum);
    uint32_t t = 0;
    for (int w = 0; w < kLT / 64; ++w) t += sm.wsum[w];
    total = t;
    __syncthreads();   // before wsum is used again
    return incl;
  };

  // 1. the first k finite logits fill slots 0..k-1 in index order: thread t
  // counts the finite logits of its span, a block prefix gives its first slot
  if (tid == 0) sm.fill_end = V;
  const int span = (V + kLT - 1) / kLT;
  const int e0 = min(V, tid * span), e1 = min(V, e0 + span);
  uint32_t nfin = 0;
  for (int e = e0; e < e1; ++e) nfin += f2key(rowp[e]) != 0u;
  uint32_t total;
  uint32_t slot = scan(nfin, total) - nfin;
  for (int e = e0; e < e1 && slot < (uint32_t)k; ++e) {
    const uint32_t key = f2key(rowp[e]);
    if (key) {
      keys[slot] = key;
      ids[slot] = e;
      if (slot == (uint32_t)k - 1) sm.fill_end = e + 1;
      ++slot;
    }
  }
  const int filled = total < (uint32_t)k ? (int)total : k;
  for (int s = filled + tid; s < k; s += kLT) { keys[s] = 0u; ids[s] = -1; }
  __syncthreads();
  const int nl1 = (k + 63) >> 6, nl2 = (nl1 + 63) >> 6, nl3 = (nl2 + 63) >> 6;   // nl3 <= 64
  for (int b = wave; b < nl1; b += kLT / 64) {
    const int sl = 64 * b + lane;
    const unsigned long long m = wave_min64(sl < k ? slot_pack(keys[sl], (uint32_t)sl) : kNone);
    if (lane == (b & 63)) lvl1[b] = m;   // the lane that reads it in the replay
  }
  __syncthreads();
  for (int c = wave; c < nl2; c += kLT / 64) {
    const int i = 64 * c + lane;
    const unsigned long long m = wave_min64(i < nl1 ? lvl1[i] : kNone);
    if (lane == 0) sm.lvl2[c] = m;
  }
  __syncthreads();
  if (wave == 0) {
    for (int d = 0; d < nl3; ++d) {
      const int i = 64 * d + lane;
      const unsigned long long m = wave_min64(i < nl2 ? sm.lvl2[i] : kNone);
      if (lane == 0) sm.lvl3[d] = m;
    }
    const unsigned long long m = wave_min64(lane < nl3 ? sm.lvl3[lane] : kNone);
    if (lane == 0) sm.root = m;
  }
  __syncthreads();

  // 2. the rest of the row, in index order: the logits above the chunk's
  // starting minimum queue up, and wave 0 takes them one by one
  const int start = sm.fill_end;
  for (int base = start; base < V; base += kLT) {
    const uint32_t lo = (uint32_t)(sm.root >> 32);
    const int e = base + tid;
    const uint32_t key = e < V ? f2key(rowp[e]) : 0u;
    const bool enter = key > lo;
    const uint32_t incl = scan(enter ? 1u : 0u, total);
    if (enter) sm.buf[incl - 1] = slot_pack(key, (uint32_t)e);
    const int nq = (int)total;
    __syncthreads();
    if (wave == 0) {
      unsigned long long top = sm.root;
      for (int q = 0; q < nq; ++q) {
        const unsigned long long item = sm.buf[q];
        const uint32_t kv = (uint32_t)(item >> 32);
        if (kv <= (uint32_t)(top >> 32)) continue;   // not above the current minimum
        const int s = (int)(uint32_t)top;
        const int b1 = s >> 6, sl = 64 * b1 + lane;
        if (sl == s) {
          keys[s] = kv;
          ids[s] = (int32_t)(uint32_t)item;
        }
        const int b2 = b1 >> 6, i1 = 64 * b2 + lane;
        // both device reads go out before the first minimum
        const uint32_t ks = sl == s ? kv : (sl < k ? keys[sl] : 0u);
        const unsigned long long l1 = i1 < nl1 && i1 != b1 ? lvl1[i1] : kNone;
        const unsigned long long m1 = wave_min64(sl < k ? slot_pack(ks, (uint32_t)sl) : kNone);
        const unsigned long long m2 = wave_min64(i1 == b1 ? m1 : l1);
        if (i1 == b1) lvl1[b1] = m1;
        const int b3 = b2 >> 6, i2 = 64 * b3 + lane;
        const unsigned long long m3 =
            wave_min64(i2 < nl2 ? (i2 == b2 ? m2 : sm.lvl2[i2]) : kNone);
        const unsigned long long m4 =
            wave_min64(lane < nl3 ? (lane == b3 ? m3 : sm.lvl3[lane]) : kNone);
        if (lane == 0) {
          sm.lvl2[b2] = m2;
          sm.lvl3[b3] = m3;
        }
        top = m4;
      }
      if (lane == 0) sm.root = top;
    }
    __syncthreads();
  }

  // 3. the token: the member of the drawn value at its rank in slot order
  const int sspan = (k + kLT - 1) / kLT;
  const int s0 = min(k, tid * sspan), s1 = min(k, s0 + sspan);
  if (req.need & 1) {
    uint32_t above = 0, eq = 0;
    for (int s = s0; s < s1; ++s) {
      const uint32_t key = keys[s];
      above += key > req.xkey;
      eq += key == req.xkey;
    }
    uint32_t n_above, n_eq;
    (void)scan(above, n_above);
    const uint32_t incl = scan(eq, n_eq);
    const int j = req.pos - (int)n_above;     // rank in the group
    if (tid == 0) sm.res = -1;
    __syncthreads();
    uint32_t seen = incl - eq;
    if (j >= 0 && (uint32_t)j >= seen && (uint32_t)j < incl) {
      for (int s = s0; s < s1; ++s) {
        if (keys[s] == req.xkey) {
          if (seen == (uint32_t)j) { sm.res = ids[s]; break; }
          ++seen;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      put_token(a, row, sm.res);
      if (sm.res < 0 && a.row_flags) a.row_flags[row] |= HS_ROW_UNSUPPORTED;
    }
    __syncthreads();
  }

  // 4. the candidate ids of positions 0..mo-1 (value descending, slot
  // ascending): the slots above X = the key at position mo - 1, and the
  // first of those equal to X in slot order, sorted
  if ((req.need & 2) && a.cand_ids) {
    const int mo = req.mo;
    const uint32_t X = req.ckey;   // >= 1: a finite logit's key
    int P2 = 1;
    while (P2 < mo) P2 <<= 1;
    for (int i = tid; i < P2; i += kLT) sm.buf[i] = 0ull;
    uint32_t gt = 0, eq = 0;
    for (int s = s0; s < s1; ++s) {
      const uint32_t key = keys[s];
      gt += key > X;
      eq += key == X;
    }
    uint32_t n_gt, n_eq;
    const uint32_t ig = scan(gt, n_gt);   // its barriers order the clearing above
    const uint32_t ie = scan(eq, n_eq);
    uint32_t pg = ig - gt, pe = ie - eq;
    for (int s = s0; s < s1; ++s) {
      const uint32_t key = keys[s];
      if (key > X) {
        if (pg < (uint32_t)mo) sm.buf[pg] = pack_cand(key, (uint32_t)s);
        ++pg;
      } else if (key == X) {
        if (n_gt + pe < (uint32_t)mo) sm.buf[n_gt + pe] = pack_cand(key, (uint32_t)s);
        ++pe;
      }
    }
    __syncthreads();
    block_sort_desc<kLT>(sm.buf, P2);
    const int cs = a.cand_stride;
    for (int i = tid; i < mo; i += kLT) {
      const unsigned long long c = sm.buf[i];   // 0: no slot (never, for a consistent request)
      a.cand_ids[(int64_t)row * cs + i] = c ? ids[cand_idx(c)] : -1;
    }
  }
  __syncthreads();   // the region and LDS are reused by the next row
}

__global__ __launch_bounds__(kLT) void large_replay_dev_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long rdyn[];
  ReplayDevSmem &sm = *reinterpret_cast<ReplayDevSmem *>(rdyn);
  const int tid = threadIdx.x, G = (int)gridDim.x, g = (int)blockIdx.x;
  uint32_t *keys = ws.replay_keys + (int64_t)g * a.vocab;
  int32_t *ids = ws.replay_ids + (int64_t)g * a.vocab;
  unsigned long long *lvl1 = ws.replay_lvl1 + (int64_t)g * ((a.vocab + 63) / 64);
  int seen = 0;   // requesting rows in the list chunks before this one
  for (int c0 = 0; c0 < a.n_large; c0 += kLT) {
    const int i = c0 + tid;
    const bool f = i < a.n_large && (ws.large_replay[i].need & kReplayDev) != 0;
    const uint32_t incl = block_scan_incl<kLT>(f ? 1u : 0u, sm.wsum);
    uint32_t total = 0;
    for (int w = 0; w < kLT / 64; ++w) total += sm.wsum[w];
    // this workgroup's ranks in the chunk: r = seen + incl - 1 with r % G == g
    const int r = seen + (int)incl - 1;
    const int first = seen + ((g - seen % G) + G) % G;   // the first such rank >= seen
    if (f && r % G == g) sm.rows[(r - first) / G] = i;
    const int mine = first < seen + (int)total ? (seen + (int)total - 1 - first) / G + 1 : 0;
    seen += (int)total;
    __syncthreads();
    for (int j = 0; j < mine; ++j) {
      const int li = sm.rows[j];
      replay_dev_row(a, ws, ws.large_replay[li], ws.large_list[li], keys, ids, lvl1, sm);
    }
    __syncthreads();   // sm.rows and wsum are rewritten by the next chunk
  }
}

// ---------------------------------------------------------------- large-k, two passes

// Rows with k = vocab (topK = Infinity or >= vocab: no slot is ever evicted,
// so the order is value descending, index ascending), no min-p and no
// candidate outputs: the common form of "top-p only" sampling.  Two passes
// over the row instead of the general path's four to six:
//
//  1. (HBM) m0 = the maximum of the first 16384 logits.  Every candidate
//     v <= m0 adds w = 2^(q * -log2(e) / 256) to bucket floor(q) of an LDS
//     histogram (64-bit fixed-point sums), q = (m0 - v) * 256 / T in binary32
//     (shared by the bucket and the weight); the few v > m0 go to a list
//     of their own.  m = max(m0, list), S = e^((m0 - m)/T) * sum + the
//     list's exp((v - m)/T).
//  2. From the buckets' cumulative probabilities the kernel picks the bucket
//     range that holds the top-p crossing and the one that holds the draw
//     (each widened where a bucket edge lies within kFEps of its target),
//     streams the row once more gathering only the logits of those buckets,
//     sorts them and walks them with exact probabilities
//     f32(f32(exp((v - m)/T)) / S) from the bucket sums before them.
//
// q's binary32 roundings and the hardware exp2 leave each weight within a few
// 1e-7 of exp((v - m0)/T), and the cumulative sums within about 1e-7 of the
// reference's sequential ones: a position can differ from the reference's
// only when its target lies that close to a cumulative boundary.  Rows the
// histogram does not suit (a non-finite maximum or temperature, fewer than
// two candidates, more than kFTop logits above m0, a crossing in the last
// bucket or none, more than kFCap gathered logits) are handed back to
// large_row.
constexpr int kFT = 1024;             // threads per workgroup
constexpr int kFB = 8192;             // buckets of 1/256 in (m0 - v) / T
constexpr float kFBScale = 256.0f;
constexpr int kFTop = 1024;           // logits above m0
constexpr int kFSpan = 2048;          // buckets of one gathered range
constexpr int kFCap = 2048;           // logits gathered for the walks
constexpr double kFEps = 1e-6;        // margin around a bucket edge (probability)

struct FastSmem {
  double mass[kFB];
  unsigned long long top[kFTop];
  unsigned long long buf[kFCap];
  double pb[kFCap];
  double dred[kFT / 64];
  unsigned long long ured[kFT / 64];
  double top_m, top_s;                 // the list's maximum and exp sum
  int ntop, nbuf, hit, flag;
  int next1, next2;                    // the passes' next unit
};

size_t large_fast_smem_bytes() { return sizeof(FastSmem); }
static_assert(kFT * 8 == kFB, "each thread owns eight buckets");

// Bucket of a candidate v <= m0 from q = (m0 - v) * 256 / T, computed once
// per logit as (m0 - v) * cz: two roundings, each relative to q itself, so
// q's error vanishes where the weights matter (small q).  (A product m0 * cz
// rounded once per row and an fma would shift every q by the same error, up
// to half an ulp of m0 * cz: a common bias of all bucket weights that grows
// with m0 / T.)  q never increases with v, so neither does the bucket;
// clamped to the last bucket.
__device__ __forceinline__ float fast_q(float v, float cz, float m0) { return (m0 - v) * cz; }
__device__ __forceinline__ int fast_bucket_q(float q) {
  return (int)fminf(fmaxf(q, 0.0f), (float)(kFB - 1));
}
__device__ __forceinline__ int fast_bucket(float v, float cz, float m0) {
  return fast_bucket_q(fast_q(v, cz, m0));
}

template <typename T>
__device__ __forceinline__ T fast_block_sum(T x, T *red) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) x += __shfl_xor(x, m);
  if (lane_id() == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  T r = 0;
  for (int w = 0; w < kFT / 64; ++w) r += red[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float fast_block_max(float x, double *red) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float y = __shfl_xor(x, m);
    x = y > x ? y : x;
  }
  if (lane_id() == 0) red[threadIdx.x >> 6] = (double)x;
  __syncthreads();
  float r = -INFINITY;
  for (int w = 0; w < kFT / 64; ++w) r = (float)red[w] > r ? (float)red[w] : r;
  __syncthreads();
  return r;
}

// In place, mass[b] becomes the sum of buckets 0..b.  Wave w owns buckets
// [512 w, 512 w + 512), read 64 consecutive at a time (no bank conflicts).
__device__ __forceinline__ void fast_prefix(FastSmem &sm) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  constexpr int per = kFB / (kFT / 64);
  double carry = 0;
#pragma unroll
  for (int i = 0; i < per / 64; ++i) {
    const int b = per * wave + 64 * i + lane;
    const double c = wave_scan_incl_f64(sm.mass[b]) + carry;
    sm.mass[b] = c;
    carry = readlane_f64(c, 63);
  }
  if (lane == 0) sm.dred[wave] = carry;
  __syncthreads();
  double base = 0;
  for (int w = 0; w < wave; ++w) base += sm.dred[w];
#pragma unroll
  for (int i = 0; i < per / 64; ++i) sm.mass[per * wave + 64 * i + lane] += base;
  __syncthreads();
}

// The first bucket b (-1: the list above m0) whose cumulative probability
// top_total + scale * mass[b] reaches x, kFB when none does.  Each wave
// searches alone, 64 probes per round (8192 -> 128 -> 2 -> 1): no barrier.
__device__ __forceinline__ int fast_first_reaching(double x, double top_total, double scale,
                                                   const FastSmem &sm) {
  if (top_total >= x) return -1;
  const int lane = lane_id();
  int base = 0, width = kFB;
  while (width > 1) {
    const int step = width >= 64 ? width / 64 : 1;
    const int idx = base + (lane + 1) * step - 1;
    const bool ok = lane * step < width && top_total + scale * sm.mass[idx] >= x;
    const unsigned long long m = __ballot(ok);
    if (!m) return width == kFB ? kFB : base + width;   // (the level above guarantees a hit)
    base += __builtin_ctzll(m) * step;
    width = step;
  }
  return base;
}

// The cumulative probability before bucket b (b = -1: 0).
__device__ __forceinline__ double fast_start(int b, double top_total, double scale,
                                             const FastSmem &sm) {
  if (b < 0) return 0.0;
  return top_total + (b > 0 ? scale * sm.mass[b - 1] : 0.0);
}

// Scratch of the walks, in the bucket array once the ranges are chosen.
struct FastWalk {
  double bsum[kFSpan];                 // exact probability per bucket of a range
  uint32_t bcnt[kFSpan];               // logits per bucket of a range
  unsigned long long one[kFCap];       // the logits of the located bucket
  double pone[kFCap];                  // their probabilities, then cumulative sums
  double ssum[16];                     // the located bucket in 16 parts: probability,
  uint32_t scnt[16];                   //   logits
  unsigned long long few[64];          // the logits of the located part
  double fewp[64];                     //   and their probabilities (wave walk)
  unsigned long long srt[64];          // the wave walk's ranked logits,
  double srp[64];                      //   and their probabilities
  int res_id, res_pos;
  double res_cum;
};
static_assert(sizeof(FastWalk) <= sizeof(double) * kFB, "the walks fit the bucket array");

// Located position in a gathered range.
struct FastLoc {
  int id;          // logit index (-1: not found)
  int pos;         // position within the range (logits of earlier buckets first)
  double cum;      // cumulative probability through it
};

// Within the range of buckets [glo, ghi] (-1: the list above m0), whose
// logits are among the nl gathered entries buf / pb (probabilities) and
// whose cumulative probability before its first logit is c_start: the first
// logit, in the reference's order (value descending, index ascending), whose
// cumulative probability reaches `target`.  The probabilities are summed
// exactly per bucket (binary64 sums of binary32 values), only the located
// bucket's logits are sorted, and the walk through them is a block prefix sum.
__device__ __forceinline__ FastLoc fast_locate(int glo, int ghi, double c_start, double target,
                                               int nl, float cz, float m0, double md,
                                               double it, double S, FastSmem &sm) {
  FastWalk &w = *reinterpret_cast<FastWalk *>(sm.mass);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int span = ghi - glo + 1;
  FastLoc r{-1, 0, 0.0};
  for (int i = tid; i < span; i += kFT) { w.bsum[i] = 0.0; w.bcnt[i] = 0u; }
  __syncthreads();
  for (int i = tid; i < nl; i += kFT) {
    const float v = key2f(cand_key(sm.buf[i]));
    const int b = v > m0 ? -1 : fast_bucket(v, cz, m0);
    if (b >= glo && b <= ghi) {
      atomicAdd(&w.bsum[b - glo], sm.pb[i]);
      atomicAdd(&w.bcnt[b - glo], 1u);
    }
  }
  __syncthreads();
  // exclusive prefix over the range's buckets: thread t owns buckets 2t, 2t+1
  static_assert(2 * kFT == kFSpan, "two buckets per thread");
  const double m0s = 2 * tid < span ? w.bsum[2 * tid] : 0.0;
  const double m1s = 2 * tid + 1 < span ? w.bsum[2 * tid + 1] : 0.0;
  const uint32_t n0 = 2 * tid < span ? w.bcnt[2 * tid] : 0u;
  const uint32_t n1 = 2 * tid + 1 < span ? w.bcnt[2 * tid + 1] : 0u;
  double cm = wave_scan_incl_f64(m0s + m1s);
  uint32_t cn = n0 + n1;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t t = __shfl_up(cn, d);
    if (lane >= d) cn += t;
  }
  if (lane == 63) { sm.dred[wave] = cm; sm.ured[wave] = cn; }
  if (tid == 0) sm.hit = 0x7FFFFFFF;
  __syncthreads();
  double bm = c_start;
  uint32_t bn = 0;
  for (int q = 0; q < wave; ++q) { bm += sm.dred[q]; bn += (uint32_t)sm.ured[q]; }
  const double e0 = bm + cm - (m0s + m1s);   // cumulative before bucket 2t
  const uint32_t k0 = bn + cn - (n0 + n1);
  if (2 * tid < span && n0 && e0 + m0s >= target) atomicMin(&sm.hit, 2 * tid);
  else if (2 * tid + 1 < span && n1 && e0 + m0s + m1s >= target) atomicMin(&sm.hit, 2 * tid + 1);
  __syncthreads();
  const int lb = sm.hit;
  if (lb >= span) { __syncthreads(); return r; }
  // the located bucket's cumulative start and position, from its owner
  if (tid == (lb >> 1)) {
    sm.dred[0] = (lb & 1) ? e0 + m0s : e0;
    sm.ured[0] = (lb & 1) ? k0 + n0 : k0;
    sm.flag = (int)((lb & 1) ? n1 : n0);
    sm.nbuf = 0;
  }
  __syncthreads();
  const double cb = sm.dred[0];
  const int kb = (int)sm.ured[0];
  const int nb = sm.flag;
  // its logits
  const int bq = glo + lb;   // the bucket (-1: the list above m0)
  for (int i = tid; i < nl; i += kFT) {
    const float v = key2f(cand_key(sm.buf[i]));
    const int b = v > m0 ? -1 : fast_bucket(v, cz, m0);
    if (b == bq) w.one[atomicAdd(&sm.nbuf, 1)] = sm.buf[i];
  }
  if (tid < 16) { w.ssum[tid] = 0.0; w.scnt[tid] = 0u; }
  if (tid == 0) w.res_id = -2;
  __syncthreads();
  auto prob = [&](unsigned long long c) {
    return (double)(float)((double)(float)exp(((double)key2f(cand_key(c)) - md) * it) / S);
  };
  // A bucket of more than 64 logits is cut in 16 parts by (q - bq) * 16,
  // clamped to [0, 15] (q - bq is exact, and the part never decreases as the
  // value falls); when the part holding the target has at most 64 logits,
  // one wave sorts and walks it.
  double cs = cb;
  int ks = kb, ns = nb;
  const unsigned long long *few = w.one;
  if (nb > 64 && bq >= 0) {
    for (int i = tid; i < nb; i += kFT) {
      const float q = fast_q(key2f(cand_key(w.one[i])), cz, m0);
      const int part = (int)fminf(fmaxf((q - (float)bq) * 16.0f, 0.0f), 15.0f);
      atomicAdd(&w.ssum[part], prob(w.one[i]));
      atomicAdd(&w.scnt[part], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      const double pm = lane < 16 ? w.ssum[lane] : 0.0;
      const uint32_t pc = lane < 16 ? w.scnt[lane] : 0u;
      const double incl = wave_scan_incl_f64(pm) + cb;
      uint32_t ci = pc;
#pragma unroll
      for (int d = 1; d < 16; d <<= 1) {
        const uint32_t t = __shfl_up(ci, d);
        if (lane >= d) ci += t;
      }
      const unsigned long long hit = __ballot(lane < 16 && pc > 0 && incl >= target);
      if (hit) {
        const int L = __builtin_ctzll(hit);
        if (lane == L) {
          sm.dred[0] = incl - pm;
          sm.ured[0] = kb + ci - pc;
          sm.flag = (int)pc;
          sm.hit = L;
        }
      } else if (lane == 0) {
        sm.flag = -1;
      }
    }
    __syncthreads();
    if (sm.flag >= 0 && sm.flag <= 64) {
      cs = sm.dred[0];
      ks = (int)sm.ured[0];
      ns = sm.flag;
      const int L = sm.hit;
      if (tid == 0) sm.nbuf = 0;
      __syncthreads();
      for (int i = tid; i < nb; i += kFT) {
        const float q = fast_q(key2f(cand_key(w.one[i])), cz, m0);
        if ((int)fminf(fmaxf((q - (float)bq) * 16.0f, 0.0f), 15.0f) == L)
          w.few[atomicAdd(&sm.nbuf, 1)] = w.one[i];
      }
      few = w.few;
    }
    __syncthreads();
  }
  if (ns <= 64) {
    // one wave: sort, probabilities, prefix sum from cs, first reaching target
    if (tid < 64) {
      unsigned long long x = lane < ns ? few[lane] : 0ull;
      x = wave_sort_desc64(x);
      const double c = wave_scan_incl_f64(lane < ns ? prob(x) : 0.0) + cs;
      const unsigned long long hit = __ballot(lane < ns && c >= target);
      if (hit) {
        const int L = __builtin_ctzll(hit);
        if (lane == L) {
          w.res_id = (int)cand_idx(x);
          w.res_pos = ks + L;
          w.res_cum = c;
        }
      } else if (lane == 0) {
        w.res_id = -1;
      }
    }
    __syncthreads();
    if (w.res_id >= 0) {
      r.id = w.res_id;
      r.pos = w.res_pos;
      r.cum = w.res_cum;
    }
    __syncthreads();
    return r;
  }
  int P2 = 1;
  while (P2 < nb) P2 <<= 1;
  for (int i = nb + tid; i < P2; i += kFT) w.one[i] = 0ull;
  __syncthreads();
  if (P2 <= 64) {
    if (tid < 64) {
      unsigned long long x = lane < P2 ? w.one[lane] : 0ull;
      x = wave_sort_desc64(x);
      if (lane < P2) w.one[lane] = x;
    }
    __syncthreads();
  } else {
    bitonic_reg<kFT, kFCap / kFT>(w.one, P2);
  }
  // their probabilities in sorted order (a function of the value alone)
  for (int i = tid; i < nb; i += kFT) {
    const float v = key2f(cand_key(w.one[i]));
    w.pone[i] = (double)(float)((double)(float)exp(((double)v - md) * it) / S);
  }
  if (tid == 0) sm.hit = 0x7FFFFFFF;
  __syncthreads();
  double carry = cb;
  for (int base = 0; base < nb; base += kFT) {
    const int i = base + tid;
    double c = wave_scan_incl_f64(i < nb ? w.pone[i] : 0.0);
    if (lane == 63) sm.dred[wave] = c;
    __syncthreads();
    double add = carry, tot = carry;
    for (int q = 0; q < kFT / 64; ++q) {
      if (q < wave) add += sm.dred[q];
      tot += sm.dred[q];
    }
    __syncthreads();
    c += add;
    if (i < nb && c >= target) atomicMin(&sm.hit, i);
    if (i < nb) w.pone[i] = c;
    carry = tot;
  }
  __syncthreads();
  const int h = sm.hit;
  if (h < nb) {
    r.id = (int)cand_idx(w.one[h]);
    r.pos = kb + h;
    r.cum = w.pone[h];
  }
  __syncthreads();
  return r;
}

// fast_locate by one wave, without a barrier, for ranges of at most 64
// buckets: the same steps (bucket sums, the located bucket, its 16 parts
// when it holds more than 64 logits, the walk through the part holding the
// target) over the probabilities in sm.pb.  The walk orders at most 64
// logits by rank (the count of larger packed keys; keys are distinct) instead
// of a sorting network.  Every lane returns the result; id -2: a part of more
// than 64 logits (or more than 64 logits above m0), which the block version
// sorts whole.  Its scratch is the bucket array's (FastWalk), as the block
// version's.
constexpr int kFWaveList = 1024;   // gathered logits the wave walks scan
__device__ __forceinline__ FastLoc fast_locate_wave(int glo, int ghi, double c_start,
                                                    double target, int nl, float cz, float m0,
                                                    FastSmem &sm) {
  FastWalk &w = *reinterpret_cast<FastWalk *>(sm.mass);
  const int lane = lane_id();
  const int span = ghi - glo + 1;
  FastLoc r{-1, 0, 0.0};
  auto bucket_of = [&](unsigned long long c) {
    const float v = key2f(cand_key(c));
    return v > m0 ? -1 : fast_bucket(v, cz, m0);
  };
  auto part_of = [&](unsigned long long c, int bq) {
    const float q = fast_q(key2f(cand_key(c)), cz, m0);
    return (int)fminf(fmaxf((q - (float)bq) * 16.0f, 0.0f), 15.0f);
  };
  // LDS operations of one wave take effect in issue order: no waits needed.
  // Loops read four entries per lane before using any.
  w.bsum[lane] = 0.0;
  w.bcnt[lane] = 0u;
  for (int base = 0; base < nl; base += 256) {
    unsigned long long c[4];
    double p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = base + 64 * k + lane;
      c[k] = i < nl ? sm.buf[i] : 0ull;
      p[k] = i < nl ? sm.pb[i] : 0.0;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int b = base + 64 * k + lane < nl ? bucket_of(c[k]) : glo - 1;
      if (b >= glo && b <= ghi) {
        atomicAdd(&w.bsum[b - glo], p[k]);
        atomicAdd(&w.bcnt[b - glo], 1u);
      }
    }
  }
  const double bs = lane < span ? w.bsum[lane] : 0.0;
  const uint32_t bc = lane < span ? w.bcnt[lane] : 0u;
  const double incl = wave_scan_incl_f64(bs);
  const uint32_t cincl = wave_scan_incl(bc);
  const double up = __shfl_up(incl, 1);
  const double before = c_start + (lane > 0 ? up : 0.0);
  const unsigned long long hb = __ballot(lane < span && bc > 0 && before + bs >= target);
  if (!hb) return r;
  const int lb = __builtin_ctzll(hb);
  const double cb = readlane_f64(before, lb);
  const int nb = (int)readlane_u32(bc, lb);
  const int kb = (int)readlane_u32(cincl, lb) - nb;
  const int bq = glo + lb;
  // the located bucket's logits and probabilities, in list order
  int n = 0;
  for (int base = 0; base < nl; base += 256) {
    unsigned long long c[4];
    double p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = base + 64 * k + lane;
      c[k] = i < nl ? sm.buf[i] : 0ull;
      p[k] = i < nl ? sm.pb[i] : 0.0;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool in = base + 64 * k + lane < nl && bucket_of(c[k]) == bq;
      const unsigned long long m = __ballot(in);
      if (in) {
        const int o = n + (int)lanes_below(m);
        w.one[o] = c[k];
        w.pone[o] = p[k];
      }
      n += __popcll(m);
    }
  }
  double cs = cb;
  int ks = kb, ns = nb;
  const unsigned long long *fx = w.one;
  const double *fp = w.pone;
  if (nb > 64) {
    if (bq < 0) { r.id = -2; return r; }
    // 16 parts by (q - bq) * 16, as the block version cuts them
    if (lane < 16) { w.ssum[lane] = 0.0; w.scnt[lane] = 0u; }
    for (int base = 0; base < nb; base += 256) {
      unsigned long long c[4];
      double p[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = base + 64 * k + lane;
        c[k] = i < nb ? w.one[i] : 0ull;
        p[k] = i < nb ? w.pone[i] : 0.0;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (base + 64 * k + lane < nb) {
          const int part = part_of(c[k], bq);
          atomicAdd(&w.ssum[part], p[k]);
          atomicAdd(&w.scnt[part], 1u);
        }
      }
    }
    const double pm = lane < 16 ? w.ssum[lane] : 0.0;
    const uint32_t pc = lane < 16 ? w.scnt[lane] : 0u;
    const double pincl = wave_scan_incl_f64(pm) + cb;
    const uint32_t ci = wave_scan_incl(pc);
    const unsigned long long hp = __ballot(lane < 16 && pc > 0 && pincl >= target);
    if (!hp) { r.id = -2; return r; }   // the block version walks the whole bucket
    const int L = __builtin_ctzll(hp);
    const int np = (int)readlane_u32(pc, L);
    if (np > 64) { r.id = -2; return r; }
    cs = readlane_f64(pincl - pm, L);
    ks = kb + (int)readlane_u32(ci, L) - np;
    ns = np;
    int f = 0;
    for (int base = 0; base < nb; base += 64) {
      const int i = base + lane;
      const unsigned long long c = i < nb ? w.one[i] : 0ull;
      const bool in = i < nb && part_of(c, bq) == L;
      const unsigned long long m = __ballot(in);
      if (in) {
        const int o = f + (int)lanes_below(m);
        w.few[o] = c;
        w.fewp[o] = w.pone[i];
      }
      f += __popcll(m);
    }
    fx = w.few;
    fp = w.fewp;
  }
  // the walk: value descending, index ascending (packed key descending)
  const unsigned long long x = lane < ns ? fx[lane] : 0ull;
  const double px = lane < ns ? fp[lane] : 0.0;
  int rank = 0;
  for (int j = 0; j < ns; ++j) {
    const unsigned long long y =
        ((unsigned long long)readlane_u32((uint32_t)(x >> 32), j) << 32) | readlane_u32((uint32_t)x, j);
    rank += y > x ? 1 : 0;
  }
  if (lane < ns) {
    w.srt[rank] = x;
    w.srp[rank] = px;
  }
  const unsigned long long xs = lane < ns ? w.srt[lane] : 0ull;
  const double c = wave_scan_incl_f64(lane < ns ? w.srp[lane] : 0.0) + cs;
  const unsigned long long hit = __ballot(lane < ns && c >= target);
  if (!hit) return r;
  const int L = __builtin_ctzll(hit);
  r.id = (int)readlane_u32(cand_idx(xs), L);
  r.pos = ks + L;
  r.cum = readlane_f64(c, L);
  return r;
}

// One row of the two-pass path; false (block-uniform) hands it back.
__device__ __forceinline__ bool large_fast(const LaunchArgs &a, const RowPlan &P, int row,
                                           FastSmem &sm) {
  constexpr int U = 4;   // float4 per thread per buffer; two buffers in flight
  constexpr int kW = kFT / 64;   // waves
  constexpr int kUnit = U * 64;  // float4 of one wave's buffer
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float *rowp = a.logits + (int64_t)row * a.stride;
  const int V = a.vocab;
  const int nfull = V >> 2;
  const rsrc_t r4 = make_rsrc(rowp, 16u * (uint32_t)nfull);
  const int nunits = (nfull + kUnit - 1) / kUnit;
  const double it = 1.0 / P.temperature;

  // Each pass hands the row out in units of kUnit float4 (4 KB): a wave's
  // first two are fixed (units w and kW + w), the rest come from an LDS
  // counter, one unit ahead, so that every wave streams until the row ends.
  // (With fixed shares the youngest waves of a CU ended each pass up to
  // 13 us after the others.)
  f32x4 A[U], B[U];
  // pass 1 reads cached (pass 2 reads the row again), pass 2 non-temporal
  auto load = [&](f32x4 (&t)[U], int n, auto policy) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(r4, (n * kUnit + u * 64 + lane) * 16, 0,
                                                           decltype(policy)::value);
      t[u] = f32x4{__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                   __uint_as_float(x[3])};
    }
  };
  // (lane 0 holds the unit; it is broadcast where used, a unit later, so
  // that no wave waits for its LDS operations at the grab)
  // (an increment below 2^32 - 1 is a plain add; unlike atomicAdd it is left
  // alone by the compiler's wave aggregation, which waits for the result)
  auto grab = [&](int *ctr) {
    int n = 0;
    if (lane == 0)
      n = (int)__builtin_amdgcn_atomic_inc32(reinterpret_cast<uint32_t *>(ctr), 0xFFFFFFFFu,
                                             __ATOMIC_RELAXED, "workgroup");
    return n;
  };
  using cached = std::integral_constant<int, 0>;
  using nontemporal = std::integral_constant<int, kReadNT>;
  // every read is unconditional (past the row a buffer read returns 0 and
  // touches no memory), so the compiler keeps both buffers in flight.  The
  // first two units go out first; the uniform comes through the scalar
  // cache, and the logits past the last whole float4 (needed after pass 1)
  // are read after the units, then the LDS is cleared.
  load(A, wave, cached{});
  load(B, kW + wave, cached{});
  __builtin_amdgcn_sched_barrier(0);
  const double u = load_scalar(a.uniforms + row);
  const float vtail = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(rowp, 4u * (uint32_t)V), (tid < (V & 3) ? 4 * nfull + tid : V) * 4, 0, 0));
  const float vt = tid < (V & 3) ? vtail : -INFINITY;
  for (int i = tid; i < kFB; i += kFT) sm.mass[i] = 0.0;
  if (tid == 0) { sm.ntop = 0; sm.nbuf = 0; sm.next1 = 2 * kW; sm.next2 = 2 * kW; }
  // m0: the largest of the first 4 U kFT logits, units 0 to kW - 1 (NaN is
  // never > anything)
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (wave * kUnit + u * 64 + lane < nfull) {
#pragma unroll
      for (int c = 0; c < 4; ++c) mx = A[u][c] > mx ? A[u][c] : mx;
    }
  }
  const float m0 = fast_block_max(mx, sm.dred);   // (its barriers order the clears above)
  const float cz = (float)(it * (double)kFBScale);
  if (!(m0 > -INFINITY && m0 < INFINITY && cz > 0.0f && cz < INFINITY))
    return false;   // (uniform: every thread read the same values)
  const float kq = -1.4426950408889634f / kFBScale;   // w = 2^(q kq) = e^((v - m0) / T)
  // The buckets sum w in fixed point, floor(w 2^sx) as 64-bit integers: LDS
  // adds of 64-bit integers run far faster than binary64 ones (the pass took
  // 28 us per row with binary64 adds).  w <= 1 (up to a rounding of q below
  // 0) and V < 2^nb, so sx = 63 - nb keeps every sum below 2^64; each weight
  // loses less than 2^-sx, which the margins below add.
  const int nbits = 32 - __clz(V);
  const int sx = 63 - nbits;
  const float sc_hi = __builtin_ldexpf(1.0f, sx - 32), sc_all = __builtin_ldexpf(1.0f, sx);
  // floor(w 2^sx): the high word floor(w 2^(sx-32)), the low word the rest
  // (both exact in binary32: w has 24 significant bits)
  auto fixw = [&](float w) {
    const float hf = floorf(w * sc_hi);
    const uint32_t lo = (uint32_t)fmaf(hf, -4294967296.0f, w * sc_all);
    return ((unsigned long long)(uint32_t)hf << 32) | lo;
  };
  unsigned long long *massx = reinterpret_cast<unsigned long long *>(sm.mass);

  // Per logit, without a branch: every one adds to some bucket (0 for those
  // that do not belong: NaN, -Infinity, and the rare v > m0, which go to
  // the list instead under one wave-uniform branch per float4).
  uint32_t nf = 0;
  auto add4 = [&](const f32x4 &t, int e) {
    const bool up0 = t[0] > m0, up1 = t[1] > m0, up2 = t[2] > m0, up3 = t[3] > m0;
    if (__builtin_expect(__any(up0 || up1 || up2 || up3), 0)) {
      const bool up[4] = {up0, up1, up2, up3};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (up[c]) {
          const int slot = atomicAdd(&sm.ntop, 1);
          if (slot < kFTop) sm.top[slot] = pack_cand(f2key(t[c]), (uint32_t)(e + c));
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float v = t[c];
      const bool cand = v > -INFINITY;
      nf += cand ? 1u : 0u;
      const float q = fast_q(v, cz, m0);
      const float w = __builtin_amdgcn_exp2f(q * kq);
      atomicAdd(&massx[fast_bucket_q(q)], fixw(cand && !(v > m0) ? w : 0.0f));
    }
  };
  auto process = [&](const f32x4 (&t)[U], int n) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = n * kUnit + u * 64 + lane;
      if (i < nfull) add4(t[u], 4 * i);
    }
  };
  {
    // units are taken in increasing order: once A's is past the row, so is B's
    int ua = wave, ub = kW + wave, nx = grab(&sm.next1);
    for (;;) {
      process(A, ua);
      ua = __builtin_amdgcn_readfirstlane(nx);
      nx = grab(&sm.next1);
      load(A, ua, cached{});
      process(B, ub);
      ub = __builtin_amdgcn_readfirstlane(nx);
      nx = grab(&sm.next1);
      load(B, ub, cached{});
      if (ua >= nunits) break;
    }
  }
  // pass 2's first reads go out now, under the analysis below
  load(A, wave, nontemporal{});
  load(B, kW + wave, nontemporal{});
  if (tid < (V & 3)) {   // the logits past the last whole float4
    const int e = 4 * nfull + tid;
    const float v = vt;
    if (v > -INFINITY) {
      ++nf;
      if (v > m0) {
        const int slot = atomicAdd(&sm.ntop, 1);
        if (slot < kFTop) sm.top[slot] = pack_cand(f2key(v), (uint32_t)e);
      } else {
        const float q = fast_q(v, cz, m0);
        atomicAdd(&massx[fast_bucket_q(q)], fixw(__builtin_amdgcn_exp2f(q * kq)));
      }
    }
  }
  const uint32_t n_f = fast_block_sum(nf, reinterpret_cast<uint32_t *>(sm.ured));
  const int ntop = sm.ntop;
  if (n_f <= 1 || ntop > kFTop) return false;

  // the maximum and S.  The list above m0 is short: one wave scans it.
  if (tid < 64) {
    float tmx = m0;
    for (int i = tid; i < ntop; i += 64) {
      const float v = key2f(cand_key(sm.top[i]));
      tmx = v > tmx ? v : tmx;
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
      const float y = __shfl_xor(tmx, d);
      tmx = y > tmx ? y : tmx;
    }
    const double mdw = (double)tmx;
    double st = 0;
    for (int i = tid; i < ntop; i += 64) st += exp(((double)key2f(cand_key(sm.top[i])) - mdw) * it);
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) st += __shfl_xor(st, d);
    if (tid == 0) { sm.top_m = mdw; sm.top_s = st; }
  }
  {
    // the sums back to binary64, each wave over the buckets it owns in
    // fast_prefix (a wave's LDS operations take effect in issue order)
    const double unit = __builtin_ldexp(1.0, -sx);
    constexpr int per = kFB / (kFT / 64);
#pragma unroll
    for (int i = 0; i < per / 64; ++i) {
      const int b = per * wave + 64 * i + lane;
      sm.mass[b] = (double)massx[b] * unit;
    }
  }
  fast_prefix(sm);   // (its barriers publish top_m, top_s)
  const float m = (float)sm.top_m;
  const double md = (double)m;
  const double R = exp(((double)m0 - md) * it);
  const double S = R * sm.mass[kFB - 1] + sm.top_s;
  // the list's probability mass (its own probabilities differ from these
  // binary64 quotients by their binary32 roundings only)
  const double top_total = sm.top_s / S;
  if (!(S > 0.0 && S < INFINITY)) return false;
  const double scale = R / S;   // bucket sum -> probability

  // 3. the bucket ranges of the top-p crossing and of the draw
  const double tp = P.top_p;
  // (the fixed point's loss, n_f 2^-sx, bounds its error in probability: S >= 1)
  const double eps = kFEps + (double)n_f * __builtin_ldexp(1.0, -sx);
  const int b1lo = fast_first_reaching(tp - eps, top_total, scale, sm);
  const int b1hi = fast_first_reaching(tp + eps, top_total, scale, sm);
  if (!(tp == tp) || b1hi >= kFB - 1) return false;   // no crossing, or in the clamped tail
  const double k_hi = fast_start(b1hi + 1, top_total, scale, sm) + eps;
  const double r_lo = u * (tp > 0.0 ? tp : 0.0) - 2 * eps;
  const double r_hi = u * k_hi + eps;
  if (!(r_lo == r_lo) || !(r_hi == r_hi)) return false;
  int b2lo = fast_first_reaching(r_lo, top_total, scale, sm);
  int b2hi = fast_first_reaching(r_hi, top_total, scale, sm);
  b2lo = b2lo < b1hi ? b2lo : b1hi;
  b2hi = b2hi < b1hi ? b2hi : b1hi;
  // range 0 holds the crossing, range 1 (above it, when apart) the draw;
  // ranges that touch become one, whose walks then share one cumulative sum
  int g0lo = b1lo, g0hi = b1hi, g1lo = b2lo, g1hi = b2hi;
  const bool two = b2hi < b1lo - 1;
  if (!two) { g0lo = b2lo < b1lo ? b2lo : b1lo; g1lo = 0; g1hi = -2; }

  // 4. gather the ranges' logits (the list above m0 joins them all).  This
  // is the row's last read: non-temporal.
  // The bucket tests run on q itself: b = trunc(clamp(q, 0, kFB - 1)) and
  // both ranges end below kFB - 1, so b < lo iff q < lo (lo > 0), and
  // lo <= b <= hi iff lo' <= q < hi + 1, lo' = lo or -Infinity for lo <= 0.
  // A NaN fails v <= m0; -Infinity gives q = +Infinity, in no test.
  const float fb0 = g0lo > 0 ? (float)g0lo : -INFINITY;
  const float fh0 = g0hi >= 0 ? (float)(g0hi + 1) : -INFINITY;
  const float fb1 = g1lo > 0 ? (float)g1lo : -INFINITY;
  const float fh1 = g1hi >= 0 ? (float)(g1hi + 1) : -INFINITY;
  uint32_t below0 = 0;   // candidates v <= m0 in buckets before g0lo
  // four logits per lane, without a branch per logit: the wave appends all
  // of a float4's gathered logits with one LDS atomic
  // (one ballot per comparison, combined as scalar masks: a ballot of a
  // combined condition costs two more vector instructions per logit)
  auto gather4 = [&](const f32x4 &t, int e, bool valid) {
    const unsigned long long mv = __builtin_amdgcn_ballot_w64(valid);
    unsigned long long m[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float v = t[c];
      const float q = fast_q(v, cz, m0);
      const bool le = v <= m0;
      below0 += (valid & le & (q < fb0)) ? 1u : 0u;
      const unsigned long long ok = mv & __builtin_amdgcn_ballot_w64(le);
      m[c] = ok & ((__builtin_amdgcn_ballot_w64(q >= fb0) & __builtin_amdgcn_ballot_w64(q < fh0)) |
                   (__builtin_amdgcn_ballot_w64(q >= fb1) & __builtin_amdgcn_ballot_w64(q < fh1)));
    }
    asm volatile("" : "+v"(below0));   // (counted here, not after the append below)
    if (__builtin_expect((m[0] | m[1] | m[2] | m[3]) != 0ull, 0)) {
      const int n0 = __popcll(m[0]), n1 = __popcll(m[1]), n2 = __popcll(m[2]);
      int base = 0;
      if (lane_id() == 0) base = atomicAdd(&sm.nbuf, n0 + n1 + n2 + __popcll(m[3]));
      base = __builtin_amdgcn_readfirstlane(base);
      const int off[4] = {base, base + n0, base + n0 + n1, base + n0 + n1 + n2};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if ((m[c] >> lane_id()) & 1ull) {
          const int slot = off[c] + (int)lanes_below(m[c]);
          if (slot < kFCap) sm.buf[slot] = pack_cand(f2key(t[c]), (uint32_t)(e + c));
        }
      }
    }
  };
  auto scan = [&](const f32x4 (&t)[U], int n) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = n * kUnit + u * 64 + lane;
      gather4(t[u], 4 * i, i < nfull);
    }
  };
  {
    int ua = wave, ub = kW + wave, nx = grab(&sm.next2);
    for (;;) {
      scan(A, ua);
      ua = __builtin_amdgcn_readfirstlane(nx);
      nx = grab(&sm.next2);
      load(A, ua, nontemporal{});
      scan(B, ub);
      ub = __builtin_amdgcn_readfirstlane(nx);
      nx = grab(&sm.next2);
      load(B, ub, nontemporal{});
      if (ua >= nunits) break;
    }
  }
  gather4(f32x4{vt, -INFINITY, -INFINITY, -INFINITY}, 4 * nfull + tid, tid < (V & 3));
  const uint32_t below = fast_block_sum(below0, reinterpret_cast<uint32_t *>(sm.ured));
  const int ng = sm.nbuf;
  const int nl = ng + ntop;
  if (nl > kFCap || g0hi - g0lo + 1 > kFSpan || g1hi - g1lo + 1 > kFSpan) return false;
  // the list above m0 joins the gathered logits; their probabilities as the
  // reference rounds them
  for (int i = tid; i < nl; i += kFT) {
    const unsigned long long c = i < ng ? sm.buf[i] : sm.top[i - ng];
    if (i >= ng) sm.buf[i] = c;
    sm.pb[i] = (double)(float)((double)(float)exp(((double)key2f(cand_key(c)) - md) * it) / S);
  }
  // the ranges' cumulative starts, read before the walks reuse the buckets
  const double c0 = fast_start(g0lo, top_total, scale, sm);
  const double c1 = two ? fast_start(g1lo, top_total, scale, sm) : 0.0;
  __syncthreads();
  auto finish = [&](const FastLoc &l1, const FastLoc &l2) {
    const int pos1 = (g0lo < 0 ? 0 : ntop + (int)below) + l1.pos;
    if (tid == 0) {
      put_token(a, row, l2.id);
      if (a.cand_count_out) a.cand_count_out[row] = (int)n_f;
      if (a.cutoff_out) a.cutoff_out[row] = pos1 + 1;
      if (a.row_flags) a.row_flags[row] = HS_ROW_LARGE | HS_ROW_TWO_PASS;
    }
  };

  // 5. src/sampler.ts:93-117 on the gathered ranges: the top-p crossing
  // (keptSum = cumProb through it), then the draw r = u keptSum.  Short lists
  // and narrow ranges: wave 0 alone, while the other waves wait at one
  // barrier (1: done, -1: hand the row back, 0: the block walks below).
  if (nl <= kFWaveList && g0hi - g0lo < 64 && g1hi - g1lo < 64) {
    if (tid < 64) {
      int res = -1;
      const FastLoc l1 = fast_locate_wave(g0lo, g0hi, c0, tp, nl, cz, m0, sm);
      if (l1.id == -2) {
        res = 0;
      } else if (l1.id >= 0) {
        const double r = u * l1.cum;
        if (r == r) {
          const FastLoc l2 =
              two ? fast_locate_wave(g1lo, g1hi, c1, r, nl, cz, m0, sm)
                  : fast_locate_wave(g0lo, g0hi, c0, r, nl, cz, m0, sm);
          res = l2.id == -2 ? 0 : l2.id >= 0 ? 1 : -1;
          if (res == 1) finish(l1, l2);
        }
      }
      if (tid == 0) sm.flag = res;
    }
    __syncthreads();
    const int res = sm.flag;
    if (res != 0) return res > 0;
  }
  const FastLoc l1 = fast_locate(g0lo, g0hi, c0, tp, nl, cz, m0, md, it, S, sm);
  if (l1.id < 0) return false;
  const double r = u * l1.cum;
  if (!(r == r)) return false;
  const FastLoc l2 = two ? fast_locate(g1lo, g1hi, c1, r, nl, cz, m0, md, it, S, sm)
                         : fast_locate(g0lo, g0hi, c0, r, nl, cz, m0, md, it, S, sm);
  if (l2.id < 0) return false;
  finish(l1, l2);
  return true;
}

// Rows of lfast_list; a row it cannot finish is marked in large_retry for
// large_kernel.  Unaligned rows and calls that want candidate outputs are
// all handed back.  Four waves per SIMD: one workgroup per CU.
__global__ __launch_bounds__(kFT, 4) void large_fast_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long ldyn[];
  const int row = ws.lfast_list[blockIdx.x];
  const RowPlan P = ws.plans[row];
  const bool ok = a.vec && !a.want_cands && a.vocab < (1 << 26) &&
                  large_fast(a, P, row, *reinterpret_cast<FastSmem *>(ldyn));
  if (threadIdx.x == 0) ws.large_retry[blockIdx.x] = ok ? 0 : 1;
}

// Rows of large_list (blocks [0, n_large)), then the rows large_fast_kernel
// handed back (block n_large + i takes lfast_list[i] when large_retry[i]).
__global__ __launch_bounds__(kLT) void large_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long ldyn[];
  __shared__ ReplayReq unused_req;   // the handed-back rows have k = vocab: never a replay
  int row;
  ReplayReq *req = &unused_req;
  if ((int)blockIdx.x < a.n_large) {
    row = ws.large_list[blockIdx.x];
    req = ws.large_replay + blockIdx.x;
  } else {
    const int i = (int)blockIdx.x - a.n_large;
    if (!ws.large_retry[i]) return;
    row = ws.lfast_list[i];
  }
  const RowPlan P = ws.plans[row];
  large_row(a, P, row, *reinterpret_cast<LargeSmem *>(ldyn), req);
}

// ---------------------------------------------------------------- GPU greedy route

// The engine sends greedy decoding without a repetition penalty
// (src/engine.ts:1600-1601) to the WGSL argmax (src/kernels.ts:1613-1654)
// instead of sampleLogits.  There, 256 invocations each keep the first id of
// their maximum over ids t, t + 256, ... (strict '>' from f32(-1e30)), and a
// tree reduction (stride 128 down to 1) keeps slot t against slot t + s on a
// tie.  Among equal maxima the winner is therefore the id whose low byte,
// bit-reversed, is smallest (the tree decides bit 7 of the invocation first
// and bit 0 last), then the smallest id; NaN and values at or below
// f32(-1e30) never win, and the result is 0 when no value exceeds it.  The
// kernel streams each row once, folding packed (value key, preference) maxima:
// no reduction tree, one comparison per logit.
__device__ __forceinline__ unsigned long long wgsl_cand(float v, uint32_t id) {
  const uint32_t pref = (__builtin_bitreverse32(id) & 0xFF000000u) | (id >> 8);
  return v > -1e30f ? ((unsigned long long)f2key(v) << 32) | (0xFFFFFFFFu - pref) : 0ull;
}

__device__ __forceinline__ int32_t wgsl_id(unsigned long long c) {
  if (!c) return 0;
  const uint32_t pref = 0xFFFFFFFFu - (uint32_t)c;
  return (int32_t)(((pref & 0x00FFFFFFu) << 8) | (__builtin_bitreverse32(pref) & 0xFFu));
}

// Thread tid reads the ids 4 (s + tid) + q of its part, s = fb + j * 1024,
// in increasing order; every id of one q lies in one WGSL invocation's
// stride class (4 s is a multiple of 256).  So each q keeps the first
// maximum of its ids (strict '>', as the invocation) and the slot s where it
// lies, which is wave-uniform: a compare and two selects per logit.
template <int NV>
__device__ __forceinline__ void wgsl_rd(const float (&v)[NV][4], int fb, float (&bv)[4],
                                        int (&bs)[4]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int s = fb + j * kRowThreads;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool take = v[j][q] > bv[q];   // NaN never
      bv[q] = take ? v[j][q] : bv[q];
      bs[q] = take ? s : bs[q];
    }
  }
}

// One 1024-thread workgroup per part of a row (a.split parts, as split rows
// of the row kernel; the last part to finish combines the parts' maxima).
template <bool VEC>
__global__ __launch_bounds__(kRowThreads) void argmax_kernel(LaunchArgs a, Workspace ws) {
  __shared__ unsigned long long wbest[kRowWaves];
  __shared__ int32_t last;
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform_i32(tid >> 6);
  const int S = a.split;
  const int row = (int)blockIdx.x / S, part = (int)blockIdx.x - row * S;
  const int nf4r = (a.vocab + 3) >> 2, per = (nf4r + S - 1) / S;
  const int f0 = min(nf4r, part * per), f1 = min(nf4r, f0 + per);
  const int eoff = 4 * f0, V = min(a.vocab, 4 * f1) - eoff;
  const float *rowp = a.logits + (int64_t)row * a.stride + eoff;
  RowSrc src;
  src.lim = VEC ? (V & ~3) : V;
  src.x4 = make_rsrc(rowp, 4u * (uint32_t)(V & ~3));
  src.x1 = make_rsrc(rowp, 4u * (uint32_t)V);
  const int nf4 = (V + 3) >> 2;
  float va[kRowNV][4], vb[kRowNV][4];
  load_rd<kRowNV, VEC>(va, src, 0, tid);
  load_rd<kRowNV, VEC>(vb, src, kRoundF4, tid);
  float tl[3] = {0.f, 0.f, 0.f};   // logits past the last whole float4 (VEC), thread 0
  if (VEC) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int e = src.lim + q;
      tl[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          src.x1, (tid == 0 && e < V ? e : V) * 4, 0, 0));
    }
  }
  float bv[4] = {-1e30f, -1e30f, -1e30f, -1e30f};   // as the invocation's initial value
  int bs[4] = {0, 0, 0, 0};
  for (int fb = 0; fb < nf4; fb += 2 * kRoundF4) {
    clip_rd<kRowNV>(va, fb, tid, src.lim);
    wgsl_rd<kRowNV>(va, fb, bv, bs);
    load_rd<kRowNV, VEC>(va, src, fb + 2 * kRoundF4, tid);   // past the part near its end
    if (fb + kRoundF4 >= nf4) break;
    clip_rd<kRowNV>(vb, fb + kRoundF4, tid, src.lim);
    wgsl_rd<kRowNV>(vb, fb + kRoundF4, bv, bs);
    load_rd<kRowNV, VEC>(vb, src, fb + 3 * kRoundF4, tid);
  }
  unsigned long long best = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const unsigned long long c = wgsl_cand(bv[q], (uint32_t)(eoff + 4 * (bs[q] + tid) + q));
    best = c > best ? c : best;
  }
  // the logits past the last whole float4 lie in other classes: candidates
  // of their own
  if (VEC && tid == 0) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int e = src.lim + q;
      const unsigned long long c = e < V ? wgsl_cand(tl[q], (uint32_t)(eoff + e)) : 0ull;
      best = c > best ? c : best;
    }
  }
  best = wave_max64(best);
  if (lane == 0) wbest[wave] = best;
  __syncthreads();
  unsigned long long bb = 0;
  if (tid == 0)
    for (int w = 0; w < kRowWaves; ++w) bb = wbest[w] > bb ? wbest[w] : bb;
  if (S == 1) {
    if (tid == 0) a.tokens[row] = wgsl_id(bb);
    return;
  }
  if (tid == 0) store_agent(&ws.split_meta[blockIdx.x].best, bb);
  if (split_arrive(ws, row, S, &last) && tid == 0) {
    for (int p = 0; p < S; ++p) {
      const unsigned long long b = load_agent(&ws.split_meta[row * S + p].best);
      bb = b > bb ? b : bb;
    }
    a.tokens[row] = wgsl_id(bb);
  }
}

// ---------------------------------------------------------------- lm_head GEMV that samples its rows
//
// One launch for the planar lm_head (src/engine.ts:1493-1515) and the
// sampler on its rows, for rows that are greedy or take k <= 64 candidates
// with at most the repetition penalty (hachiue's defaults: topK 20).  In the
// GEMV's loop a tile's results are only written as logits and recorded in
// the wave's LDS buffer.  After the loop each wave penalises its recorded
// results where the row's history asks for it (src/sampler.ts:24-33: the
// last 128 ids, each distinct id once; the logit is written again) and
// publishes its two largest packed candidates (value, then index: distinct)
// with the tiles it recorded; the workgroup counts its largest in the row's
// histogram of keys (kFuseHist bins of the keys' top 12 bits, in device
// memory; one atomic per workgroup: per wave they queued on the few bins
// the maxima share).  The last workgroup to count itself in reads the
// histogram and every wave's two largest in one round trip.  The
// workgroups' maxima are distinct logits of the row, so the bin b* holding
// the 64th largest of them bounds the row's 64th largest from below: every
// logit of the row's top 64 (and every logit equal to its k-th largest,
// k <= 64) lies in a bin >= b*.  Such a logit is its wave's maximum, or
// else its wave's second largest lies there too, and that wave's tiles are
// read again from the written logits.  The candidates gathered are ranked and the row kernel's
// tail runs on the top 64 (wave_tail, with the slot replay over the written
// logits when equal values decide the draw: the 65th largest candidate
// equal to the k-th, or more than kFuseStage candidates).  Greedy rows keep
// the packed maximum instead.  No workgroup waits for another: each
// publishes with agent-scope stores, waits for them, then counts itself in;
// the one that counts last reads, and clears the histogram for the next
// call.

constexpr int kFuseSetSlots = 256;   // repetition ids of a row (at most 128)
__device__ __forceinline__ uint32_t fuse_hash(int id) {
  return ((uint32_t)id * 2654435761u) >> 24;
}
__device__ __forceinline__ bool fuse_in_set(const int32_t *set, int id) {
  uint32_t h = fuse_hash(id);
  for (int probe = 0; probe < kFuseSetSlots; ++probe) {
    const int v = set[h];
    if (v == id) return true;
    if (v < 0) return false;
    h = (h + 1) & (kFuseSetSlots - 1);
  }
  return false;
}

struct FuseSmem {
  int32_t rset[kFuseSetSlots];
  unsigned long long best[16];
  uint32_t wsum[16];
  uint32_t key64;
  int32_t last, nf, bin, nmore;
  unsigned long long top[64];
  float rsv[64];
  int32_t rsid[64];
  double sp[64];
};

// The epilogue the GEMV body calls with each tile's results (tern_gemv.h):
// the logit is written through (the last workgroup may replay the row),
// except at the row's repetition ids, written once penalised after the loop,
// and (value bits, row) recorded in the wave's buffer; row ~0u marks no
// result.
struct RecordEpi {
  float *y;
  uint2 *wbuf;          // cap * 16 entries
  const int32_t *rset;  // the repetition ids, or null
  int nt;               // tiles recorded (wave-uniform)
  int cap;              // tiles the buffer holds
  __device__ __forceinline__ void out(int lane, int row, float v, bool valid) {
    if (valid && !(rset && fuse_in_set(rset, row))) store_agent(y + row, v);
    // (the launch gives no wave more than cap tiles)
    if (!__ballot(valid) || nt >= cap) return;
    if (lane < 16)
      wbuf[nt * 16 + lane] = make_uint2(__float_as_uint(v), valid ? (uint32_t)row : ~0u);
    ++nt;
  }
};

constexpr int kFuseMore = 1024;   // waves whose tiles the last workgroup reads again
// LDS: the GEMV body's, the waves' result buffers, then the list of waves
// read again, the candidates and their ranks.
size_t tern_sample_lds_bytes(int K, int nw) {
  return gemv_tern_lds_bytes(K) + (size_t)nw * kFuseTiles * 16 * sizeof(uint2) +
         (size_t)kFuseMore * sizeof(int32_t) +
         (size_t)kFuseStage * (sizeof(unsigned long long) + sizeof(int32_t));
}

// Counts the calling workgroup in at *cnt (after its published stores
// completed); true in the one that counts `of`, which also zeroes *cnt for
// the next call.  Every thread calls it.
__device__ __forceinline__ bool fuse_arrive(uint32_t *cnt, uint32_t of, FuseSmem &fs) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    fs.last = old == of - 1;
    if (fs.last) store_agent(cnt, 0u);
  }
  __syncthreads();
  return fs.last != 0;
}

// Row m's repetition set (src/sampler.ts:24-33: history.slice(-128), ids
// in [0, N)) into rset (kFuseSetSlots slots, -1 when empty, cleared by the
// caller beforehand), by threads 0-127.
__device__ __forceinline__ void fuse_rep_set(const FuseArgs &f, int m, int N, int32_t *rset) {
  const int tid = threadIdx.x;
  if (!f.hist_off || tid >= 128) return;
  const int64_t h0 = f.hist_off[m], n = f.hist_off[m + 1] - h0;
  const int64_t j = n - (n < 128 ? n : 128) + tid;
  if (j >= n) return;
  const int id = f.hist_ids[h0 + j];
  if (id < 0 || id >= N) return;
  uint32_t h = fuse_hash(id);
  for (int probe = 0; probe < kFuseSetSlots; ++probe) {
    const int old = atomicCAS(&rset[h], -1, id);
    if (old == -1 || old == id) break;
    h = (h + 1) & (kFuseSetSlots - 1);
  }
}

// After the GEMV loop of a workgroup whose waves recorded their tiles'
// results (RecordEpi: at most `tiles` tiles a wave, wave w's at
// rec + w * tiles * 16, the calling wave's count `nt`): the row's sampling,
// as described above.  `more` (kFuseMore entries) and `cand` (kFuseStage
// candidates, then kFuseStage ranks) are LDS the GEMV body no longer uses,
// disjoint from each other and from the record buffers.  Every thread calls
// it.
template <int NW>
__device__ void fuse_sample_finish(const GemvArgs &g, const FuseArgs &f, int m, int nt, int tiles,
                                   const uint2 *rec, int32_t *more, unsigned long long *cand,
                                   FuseSmem &fs) {
  constexpr int NT = 64 * NW;
  constexpr int HB = kFuseHist / NT;        // histogram bins a thread reads
  constexpr int WPT = kFuseWavesPerThread;  // waves' entries a thread reads
  static_assert(kFuseHist % NT == 0, "whole bins per thread");
  // ---- this wave's results as packed candidates (penalties applied): its
  // maximum, and for sampling rows its second largest too
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const RowPlan *plan = f.plans + m;
  const int mode = load_scalar(&plan->mode);
  const bool rep = (load_scalar(&plan->pen) & kPenRep) != 0;
  float *y = g.y + (int64_t)m * g.ldy;
  const uint2 *wbuf = rec + wave * tiles * 16;
  const bool greedy = mode == kModeGreedy;
  const double prep = load_scalar(&plan->rep);
  const int ne = nt * 16;
  unsigned long long m1 = 0ull, m2 = 0ull;   // this lane's largest two
  for (int e = lane; e < ne; e += 64) {
    const uint2 r = wbuf[e];
    float v = __uint_as_float(r.x);
    if (r.y == ~0u) continue;
    if (rep && fuse_in_set(fs.rset, (int)r.y)) {
      RowPlan pr{};
      pr.rep = prep;
      pr.pen = kPenRep;
      v = penalise(v, true, 0u, pr);
      store_agent(y + r.y, v);
    }
    const uint32_t key = f2key(v);
    const unsigned long long c = key ? pack_cand(key, r.y) : 0ull;
    if (c > m1) {
      m2 = m1;
      m1 = c;
    } else if (c > m2) {
      m2 = c;
    }
  }
  FuseRow *fr = f.rows + m;
  LaunchArgs a{};
  a.logits = g.y;
  a.stride = g.ldy;
  a.rows = g.M;
  a.vocab = g.N;
  a.uniforms = f.uniforms;
  a.tokens = f.tokens;

  if (greedy) {   // the packed maximum; the last workgroup writes the token
    const unsigned long long b = wave_max64(m1);
    if (lane == 0) fs.best[wave] = b;
    __syncthreads();
    if (tid == 0) {
      unsigned long long bb = 0ull;
      for (int w = 0; w < NW; ++w) bb = fs.best[w] > bb ? fs.best[w] : bb;
      if (bb) __hip_atomic_fetch_max(&fr->best, bb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!fuse_arrive(&fr->arrived, gridDim.x, fs)) return;
    if (tid == 0) {
      const unsigned long long bb = load_agent(&fr->best);
      write_greedy(a, m, load_agent(y), bb);
      store_agent(&fr->best, 0ull);
    }
    return;
  }

  // ---- the wave's two largest (distinct: the index is packed in) and its
  // tiles; the workgroup's largest counted in the row's histogram
  const int Bw = f.blocks * NW;
  unsigned long long *wx0 = f.wtop + (int64_t)m * 2 * Bw, *wx1 = wx0 + Bw;
  int32_t *wt = f.wtiles + (int64_t)m * Bw * kFuseTileWords;
  uint32_t *hist = f.hist + (int64_t)m * kFuseHist;
  {
    const unsigned long long x0 = wave_max64(m1);
    const unsigned long long x1 = wave_max64(m1 == x0 ? m2 : m1);
    const int wg = (int)blockIdx.x * NW + wave;
    if (lane == 0) {
      store_agent(wx0 + wg, x0);
      store_agent(wx1 + wg, x1);
      fs.best[wave] = x0;
    }
    // [0]: the count; [1 + e]: tile e, whose first lane holds its first row
    if (lane <= nt)
      store_agent(wt + (int64_t)wg * kFuseTileWords + lane,
                  lane == 0 ? nt : (int32_t)(wbuf[(lane - 1) * 16].y >> 4));
    __syncthreads();
    if (tid == 0) {
      unsigned long long bb = 0ull;
      for (int w = 0; w < NW; ++w) bb = fs.best[w] > bb ? fs.best[w] : bb;
      if (bb)
        __hip_atomic_fetch_add(hist + (cand_key(bb) >> 20), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!fuse_arrive(&fr->arrived, (uint32_t)f.blocks, fs)) return;

  // ---- the row, by the last workgroup: the histogram and the waves' two
  // largest in one round trip
  uint32_t hc[HB];
  unsigned long long w0[WPT], w1[WPT];
#pragma unroll
  for (int i = 0; i < HB; ++i) hc[i] = load_agent(hist + tid * HB + i);
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int w = tid + i * NT;
    w0[i] = w < Bw ? load_agent(wx0 + w) : 0ull;
    w1[i] = w < Bw ? load_agent(wx1 + w) : 0ull;
  }
  uint32_t tsum = 0;
#pragma unroll
  for (int i = 0; i < HB; ++i) {
    tsum += hc[i];
    store_agent(hist + tid * HB + i, 0u);   // zero for the next call
  }
  if (tid == 0) { fs.bin = 0; fs.nf = 0; fs.nmore = 0; fs.key64 = 0u; }
  int32_t *rnk = reinterpret_cast<int32_t *>(cand + kFuseStage);
  for (int i = tid; i < kFuseStage; i += NT) rnk[i] = 0;
  for (int i = tid; i < 64; i += NT) fs.top[i] = 0ull;
  // b*: the bin where the count of workgroup maxima from the top reaches 64
  // (0 when there are fewer); thread t holds bins t * HB .. t * HB + HB - 1
  const uint32_t incl = block_scan_incl<NT>(tsum, fs.wsum);
  uint32_t total = 0;
  for (int w = 0; w < NW; ++w) total += fs.wsum[w];
  const uint32_t above = total - incl;   // in the bins of later threads
  if (above < 64u && above + tsum >= 64u) {
    uint32_t cum = above;
#pragma unroll
    for (int i = HB - 1; i >= 0; --i) {
      cum += hc[i];
      if (cum >= 64u) {
        fs.bin = tid * HB + i;
        break;
      }
    }
  }
  __syncthreads();
  const uint32_t bstar = (uint32_t)fs.bin;
  auto in = [&](unsigned long long c) { return c != 0ull && (cand_key(c) >> 20) >= bstar; };
  auto add = [&](bool keep, unsigned long long x) {   // every lane of the wave calls it
    const unsigned long long bl = __ballot(keep);
    if (!bl) return;
    int base = 0;
    if (lane == 0) base = atomicAdd(&fs.nf, __popcll(bl));
    base = __shfl(base, 0);
    const int p = base + (int)lanes_below(bl);
    if (keep && p < kFuseStage) cand[p] = x;
  };
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    add(in(w0[i]), w0[i]);
    if (in(w1[i])) {
      const int q = atomicAdd(&fs.nmore, 1);
      if (q < kFuseMore) more[q] = tid + i * NT;
    }
  }
  __syncthreads();
  // the waves with a second logit at b* or above: their tiles again, from
  // the written logits (a few waves on common rows)
  const int nmore = fs.nmore;
  for (int q = wave; q < nmore && q < kFuseMore; q += NW) {
    const int w = more[q];
    const int32_t *tw = wt + (int64_t)w * kFuseTileWords;
    const int ntw = load_agent(tw);
    const unsigned long long x0w = load_agent(wx0 + w);   // listed already
    for (int p = 0; p < ntw; p += 4) {
      const int e = p + (lane >> 4);
      unsigned long long c = 0ull;
      if (e < ntw) {
        const int row = load_agent(tw + 1 + e) * 16 + (lane & 15);
        if (row < g.N) {
          const uint32_t key = f2key(load_agent(y + row));
          c = key ? pack_cand(key, (uint32_t)row) : 0ull;
        }
      }
      add(c != x0w && in(c), c);
    }
  }
  __syncthreads();
  const int nf = fs.nf;
  const bool ovf = nf > kFuseStage || nmore > kFuseMore;
  const int n = ovf ? 0 : nf;
  // the top 64 and the 65th: each candidate's rank is the count of larger
  // ones, split over S threads a candidate when there are few (a few
  // hundred on common rows)
  const int S = n > 0 && 2 * n <= NT ? min(16, NT / n) : 1;
  if (S > 1) {
    const int i = tid / S, sl = tid - i * S;
    if (i < n) {
      const unsigned long long xi = cand[i];
      int cnt = 0;
      for (int j = sl; j < n; j += S) cnt += cand[j] > xi ? 1 : 0;
      atomicAdd(&rnk[i], cnt);
    }
    __syncthreads();
  }
  for (int i = tid; i < n; i += NT) {
    const unsigned long long xi = cand[i];
    int rank = 0;
    if (S > 1) {
      rank = rnk[i];
    } else {
      for (int j = 0; j < n; ++j) rank += cand[j] > xi ? 1 : 0;
    }
    if (rank < 64) fs.top[rank] = xi;
    if (rank == 64) fs.key64 = cand_key(xi);
  }
  __syncthreads();
  if (wave != 0) return;
  const unsigned long long F = fs.top[lane];
  RowPlan P{};
  P.temperature = load_scalar(&plan->temperature);
  P.top_p = load_scalar(&plan->top_p);
  P.min_p = load_scalar(&plan->min_p);
  P.k = load_scalar(&plan->k);
  const uint32_t Tk = cand_key(__shfl(F, P.k - 1));
  const bool extra = Tk != 0u && fs.key64 == Tk;
  // (a replay here is rare: fewer logits in flight keep the GEMV's registers)
  finish_wave<4>(a, P, m, y, F, extra, ovf, f.uniforms[m], fs.rsv, fs.rsid, fs.sp, true);
}

// (one 16-wave workgroup per CU, as the plain GEMV)
template <int FMT>
__global__ __launch_bounds__(64 * tm::waves<FMT>()) void gemv_tern_sample_kernel(GemvArgs g,
                                                                                   FuseArgs f) {
  constexpr int NW = tm::waves<FMT>();
  extern __shared__ uint4 tlds[];
  __shared__ FuseSmem fs;
  const int tid = threadIdx.x, wave = tid >> 6;
  const int m = (int)blockIdx.y;
  const bool rep = (load_scalar(&f.plans[m].pen) & kPenRep) != 0;
  float *y = g.y + (int64_t)m * g.ldy;

  // the row's repetition set: history.slice(-128), ids in [0, N)
  if (tid < kFuseSetSlots) fs.rset[tid] = -1;
  __syncthreads();
  if (rep) fuse_rep_set(f, m, g.N, fs.rset);
  // (the body's first barrier completes the set)

  uint8_t *lb = reinterpret_cast<uint8_t *>(tlds);
  uint2 *rec = reinterpret_cast<uint2 *>(lb + gemv_tern_lds_bytes(g.K));
  RecordEpi epi{y, rec + wave * kFuseTiles * 16, rep ? fs.rset : nullptr, 0, kFuseTiles};
  tern_gemv_body<FMT>(g, tlds, epi);
  int32_t *more = reinterpret_cast<int32_t *>(rec + NW * kFuseTiles * 16);
  fuse_sample_finish<NW>(g, f, m, epi.nt, kFuseTiles, rec, more,
                         reinterpret_cast<unsigned long long *>(more + kFuseMore), fs);
}

// The fused kernel's grid: as the GEMV's (one workgroup per CU, at most one
// per tile); 0 when a wave would get more than kFuseTiles tiles or the last
// workgroup's threads more than kFuseWavesPerThread waves' entries.
template <int FMT>
int tern_sample_blocks(const GemvArgs &g, size_t lds) {
  constexpr int nw = tm::waves<FMT>();
  const int ntiles = (g.N + 15) / 16;
  const int res = resident_blocks(reinterpret_cast<const void *>(gemv_tern_sample_kernel<FMT>),
                                  (uint32_t)lds, 64 * nw);
  const int blocks = ntiles < res ? ntiles : res;
  return tern_out_tiles_max(g.N, g.K, blocks, nw) <= kFuseTiles &&
                 blocks * nw <= kFuseWavesPerThread * 64 * nw
             ? blocks
             : 0;
}

int tern_sample_grid(const GemvArgs &g) {
  switch (g.type) {
    case kW_Q1_0: return tern_sample_blocks<kW_Q1_0>(g, tern_sample_lds_bytes(g.K, tm::waves<kW_Q1_0>()));
    case kW_PQ2_0: return tern_sample_blocks<kW_PQ2_0>(g, tern_sample_lds_bytes(g.K, tm::waves<kW_PQ2_0>()));
    case kW_PTQ1_0: return tern_sample_blocks<kW_PTQ1_0>(g, tern_sample_lds_bytes(g.K, tm::waves<kW_PTQ1_0>()));
    default: return 0;
  }
}

// Every row greedy (src/sampler.ts:36-46 at temperature <= 0): the GEMV
// whose epilogue stores each logit (its repetition penalty applied, as
// pen_kernel does) and keeps each lane's packed maximum (value, then the
// smallest index); no record buffer, the plain GEMV's LDS and grid.  The
// workgroup's maximum goes to the row's word by an atomic maximum; the last
// workgroup to count in writes the token.
struct ArgmaxEpi {
  float *y;
  const int32_t *rset;   // the repetition ids, or null
  double rep;
  unsigned long long best;
  __device__ __forceinline__ void out(int, int row, float v, bool valid) {
    if (!valid) return;
    if (rset && fuse_in_set(rset, row)) {
      RowPlan pr{};
      pr.rep = rep;
      pr.pen = kPenRep;
      v = penalise(v, true, 0u, pr);
    }
    store_agent(y + row, v);
    const uint32_t key = f2key(v);
    const unsigned long long c = key ? pack_cand(key, (uint32_t)row) : 0ull;
    best = c > best ? c : best;
  }
};

// The end of an all-greedy fused GEMV (every thread calls it, after the
// body): the workgroup's packed maximum into the row's word, then the count;
// the last workgroup writes the token.
template <int NW>
__device__ __forceinline__ void fuse_argmax_finish(const GemvArgs &g, const FuseArgs &f, int m,
                                                   unsigned long long best,
                                                   unsigned long long *wbest) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float *y = g.y + (int64_t)m * g.ldy;
  const unsigned long long b = wave_max64(best);
  if (lane == 0) wbest[wave] = b;
  __syncthreads();
  FuseRow *fr = f.rows + m;
  if (tid == 0) {
    unsigned long long bb = 0ull;
    for (int w = 0; w < NW; ++w) bb = wbest[w] > bb ? wbest[w] : bb;
    if (bb) __hip_atomic_fetch_max(&fr->best, bb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // counted in after the stores and the maximum completed
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(&fr->arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1) {
      store_agent(&fr->arrived, 0u);
      LaunchArgs a{};
      a.logits = g.y;
      a.stride = g.ldy;
      a.rows = g.M;
      a.vocab = g.N;
      a.uniforms = f.uniforms;
      a.tokens = f.tokens;
      const unsigned long long bb = load_agent(&fr->best);
      write_greedy(a, m, load_agent(y), bb);
      store_agent(&fr->best, 0ull);
    }
  }
}

template <int FMT>
__global__ __launch_bounds__(64 * tm::waves<FMT>())
void gemv_tern_argmax_kernel(GemvArgs g, FuseArgs f) {
  constexpr int NW = tm::waves<FMT>();
  extern __shared__ uint4 tlds[];
  __shared__ int32_t rset[kFuseSetSlots];
  __shared__ unsigned long long wbest[NW];
  const int tid = threadIdx.x;
  const int m = (int)blockIdx.y;
  const RowPlan *plan = f.plans + m;
  const bool rep = (load_scalar(&plan->pen) & kPenRep) != 0;
  if (tid < kFuseSetSlots) rset[tid] = -1;
  __syncthreads();
  if (rep) fuse_rep_set(f, m, g.N, rset);
  // (the body's first barrier completes the set)
  ArgmaxEpi epi{g.y + (int64_t)m * g.ldy, rep ? rset : nullptr, load_scalar(&plan->rep), 0ull};
  tern_gemv_body<FMT>(g, tlds, epi);
  fuse_argmax_finish<NW>(g, f, m, epi.best, wbest);
}

// The same on the Q4_K and Q6_K bodies (the grid and LDS of the plain
// matrix-core GEMV, gemv_kq_mfma_kernel).
template <int FMT>
__global__ __launch_bounds__(KqBody<FMT>::kThreads, 2) void gemv_kq_argmax_kernel(GemvArgs g, FuseArgs f) {
  constexpr int NW = KqBody<FMT>::kWaves;
  extern __shared__ uint4 qlds[];
  __shared__ int32_t rset[kFuseSetSlots];
  __shared__ unsigned long long wbest[NW];
  const int tid = threadIdx.x;
  const int m = (int)blockIdx.y;
  const RowPlan *plan = f.plans + m;
  const bool rep = (load_scalar(&plan->pen) & kPenRep) != 0;
  if (tid < kFuseSetSlots) rset[tid] = -1;
  __syncthreads();
  if (rep) fuse_rep_set(f, m, g.N, rset);
  // (the body's first barrier completes the set)
  ArgmaxEpi epi{g.y + (int64_t)m * g.ldy, rep ? rset : nullptr, load_scalar(&plan->rep), 0ull};
  KqBody<FMT>::run(g, reinterpret_cast<uint8_t *>(qlds), epi);
  fuse_argmax_finish<NW>(g, f, m, epi.best, wbest);
}

// The same for F32, Q4_0 and Q4_1 (the vector-unit bodies, blk_gemv.h;
// LDSB: the block formats' LDS batches), on the GEMV's grid.
template <int FMT, int NRU, bool LDSB>
__global__ __launch_bounds__(kGemvThreads) void gemv_blk_argmax_kernel(GemvArgs g, FuseArgs f) {
  constexpr int NW = kGemvThreads / 64;
  extern __shared__ uint4 glds[];
  __shared__ int32_t rset[kFuseSetSlots];
  __shared__ unsigned long long wbest[NW];
  const int tid = threadIdx.x;
  const int m = (int)blockIdx.y;
  const RowPlan *plan = f.plans + m;
  const bool rep = (load_scalar(&plan->pen) & kPenRep) != 0;
  if (tid < kFuseSetSlots) rset[tid] = -1;
  __syncthreads();
  if (rep) fuse_rep_set(f, m, g.N, rset);
  __syncthreads();   // (the bodies have no barrier of their own)
  ArgmaxEpi epi{g.y + (int64_t)m * g.ldy, rep ? rset : nullptr, load_scalar(&plan->rep), 0ull};
  if constexpr (LDSB)
    gemv_lds_body<FMT, NRU>(g, glds, epi);
  else
    gemv_vec_body<FMT, NRU>(g, epi);
  fuse_argmax_finish<NW>(g, f, m, epi.best, wbest);
}

template <int FMT, int NRU>
const void *blk_argmax_fn() {
  if constexpr (FMT == kW_F32)
    return reinterpret_cast<const void *>(gemv_blk_argmax_kernel<FMT, NRU, false>);
  else
    return reinterpret_cast<const void *>(gemv_blk_argmax_kernel<FMT, NRU, true>);
}

// The block formats' grid: the GEMV's (g.blocks, at most the resident
// workgroups), and the launch.
template <int FMT, int NRU>
hipError_t launch_blk_argmax(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                             hipEvent_t *ev, hipEvent_t done, int *blocks_out) {
  const uint32_t lds = FMT == kW_F32 ? 0u : (uint32_t)gemv_lds_bytes(FMT);
  const int res = resident_blocks(blk_argmax_fn<FMT, NRU>(), lds, kGemvThreads);
  const int blocks = g.blocks < res ? g.blocks : res;
  if (blocks_out) {
    *blocks_out = blocks;
    return hipSuccess;
  }
  if (blocks < 1) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)g.M), block(kGemvThreads);
  auto go = [&](auto kern) {
    if (ev)
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, ev[0], ev[1], 0u, g, f);
    else if (done)
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, nullptr, done, 0u, g, f);
    else
      hipLaunchKernelGGL(kern, grid, block, lds, stream, g, f);
    return hipGetLastError();
  };
  if constexpr (FMT == kW_F32)
    return go(gemv_blk_argmax_kernel<FMT, NRU, false>);
  else
    return go(gemv_blk_argmax_kernel<FMT, NRU, true>);
}

// blocks_out: only the grid, nothing launched
hipError_t blk_argmax(const GemvArgs &g, const FuseArgs &f, hipStream_t stream, hipEvent_t *ev,
                      hipEvent_t done, int *blocks_out) {
  const bool two = g.nru == 2;
  switch (g.type) {
    case kW_F32: return two ? launch_blk_argmax<kW_F32, 2>(g, f, stream, ev, done, blocks_out)
                            : launch_blk_argmax<kW_F32, 1>(g, f, stream, ev, done, blocks_out);
    case kW_Q4_0: return two ? launch_blk_argmax<kW_Q4_0, 2>(g, f, stream, ev, done, blocks_out)
                             : launch_blk_argmax<kW_Q4_0, 1>(g, f, stream, ev, done, blocks_out);
    case kW_Q4_1: return two ? launch_blk_argmax<kW_Q4_1, 2>(g, f, stream, ev, done, blocks_out)
                             : launch_blk_argmax<kW_Q4_1, 1>(g, f, stream, ev, done, blocks_out);
    default: return hipErrorInvalidValue;
  }
}

template <int FMT>
int kq_argmax_grid(const GemvArgs &g) {
  using B = KqBody<FMT>;
  const int ntiles = (g.N + 15) / 16;
  const int res = resident_blocks(reinterpret_cast<const void *>(gemv_kq_argmax_kernel<FMT>),
                                  (uint32_t)B::lds(g.K), B::kThreads);
  int blocks = (ntiles + B::kWaves - 1) / B::kWaves;
  blocks = blocks < res ? blocks : res;
  blocks = blocks < g.part_cap / B::kWaves ? blocks : g.part_cap / B::kWaves;
  return blocks >= 1 && g.part && g.tile_cnt ? blocks : 0;
}

template <int FMT>
hipError_t launch_kq_argmax(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                            hipEvent_t *ev, hipEvent_t done) {
  using B = KqBody<FMT>;
  const int blocks = kq_argmax_grid<FMT>(g);
  if (blocks < 1) return hipErrorInvalidValue;
  const size_t lds = B::lds(g.K);
  const dim3 grid((unsigned)blocks, (unsigned)g.M), block(B::kThreads);
  if (ev)
    hipExtLaunchKernelGGL(gemv_kq_argmax_kernel<FMT>, grid, block, lds, stream, ev[0], ev[1], 0u, g, f);
  else if (done)
    hipExtLaunchKernelGGL(gemv_kq_argmax_kernel<FMT>, grid, block, lds, stream, nullptr, done, 0u, g, f);
  else
    hipLaunchKernelGGL(gemv_kq_argmax_kernel<FMT>, grid, block, lds, stream, g, f);
  return hipGetLastError();
}

int argmax_fused_grid(const GemvArgs &g) {
  if (g.type == kW_Q6_K) return kq_argmax_grid<kW_Q6_K>(g);
  if (g.type == kW_Q4_K) return kq_argmax_grid<kW_Q4_K>(g);
  if (tern_quant_bytes(g.type) == 0) {
    int blocks = 0;
    return blk_argmax(g, FuseArgs{}, nullptr, nullptr, nullptr, &blocks) == hipSuccess ? blocks : 0;
  }
  const int nw = g.type == kW_Q1_0 ? tm::waves<kW_Q1_0>()
                 : g.type == kW_PQ2_0 ? tm::waves<kW_PQ2_0>() : tm::waves<kW_PTQ1_0>();
  const void *k = g.type == kW_Q1_0 ? reinterpret_cast<const void *>(gemv_tern_argmax_kernel<kW_Q1_0>)
                  : g.type == kW_PQ2_0 ? reinterpret_cast<const void *>(gemv_tern_argmax_kernel<kW_PQ2_0>)
                                       : reinterpret_cast<const void *>(gemv_tern_argmax_kernel<kW_PTQ1_0>);
  const int res = resident_blocks(k, (uint32_t)gemv_tern_lds_bytes(g.K), 64 * nw);
  const int ntiles = (g.N + 15) / 16;
  return ntiles < res ? ntiles : res;
}

hipError_t launch_argmax_fused(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                               hipEvent_t *ev, hipEvent_t done) {
  auto go = [&](auto kern, int nw) {
    const int blocks = argmax_fused_grid(g);
    if (blocks < 1) return hipErrorInvalidValue;
    const size_t lds = gemv_tern_lds_bytes(g.K);
    const dim3 grid((unsigned)blocks, (unsigned)g.M), block(64 * nw);
    if (ev)
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, ev[0], ev[1], 0u, g, f);
    else if (done)
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, nullptr, done, 0u, g, f);
    else
      hipLaunchKernelGGL(kern, grid, block, lds, stream, g, f);
    return hipGetLastError();
  };
  switch (g.type) {
    case kW_Q1_0: return go(gemv_tern_argmax_kernel<kW_Q1_0>, tm::waves<kW_Q1_0>());
    case kW_PQ2_0: return go(gemv_tern_argmax_kernel<kW_PQ2_0>, tm::waves<kW_PQ2_0>());
    case kW_PTQ1_0: return go(gemv_tern_argmax_kernel<kW_PTQ1_0>, tm::waves<kW_PTQ1_0>());
    case kW_Q6_K: return launch_kq_argmax<kW_Q6_K>(g, f, stream, ev, done);
    case kW_Q4_K: return launch_kq_argmax<kW_Q4_K>(g, f, stream, ev, done);
    default: return blk_argmax(g, f, stream, ev, done, nullptr);
  }
}

hipError_t launch_tern_sample(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                              hipEvent_t *ev, hipEvent_t done) {
  auto go = [&](auto kern, int nw, int blocks) {
    if (blocks < 1) return hipErrorInvalidValue;
    const size_t lds = tern_sample_lds_bytes(g.K, nw);
    const dim3 grid((unsigned)blocks, (unsigned)g.M), block(64 * nw);
    if (ev)
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, ev[0], ev[1], 0u, g, f);
    else if (done)
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, nullptr, done, 0u, g, f);
    else
      hipLaunchKernelGGL(kern, grid, block, lds, stream, g, f);
    return hipGetLastError();
  };
  const int blocks = tern_sample_grid(g);
  if (blocks != f.blocks) return hipErrorInvalidValue;   // the workspace was sized for another grid
  switch (g.type) {
    case kW_Q1_0: return go(gemv_tern_sample_kernel<kW_Q1_0>, tm::waves<kW_Q1_0>(), blocks);
    case kW_PQ2_0: return go(gemv_tern_sample_kernel<kW_PQ2_0>, tm::waves<kW_PQ2_0>(), blocks);
    case kW_PTQ1_0: return go(gemv_tern_sample_kernel<kW_PTQ1_0>, tm::waves<kW_PTQ1_0>(), blocks);
    default: return hipErrorInvalidValue;
  }
}

// ---- the Q4_K and Q6_K lm_head GEMVs that sample their rows
//
// gemv_tern_sample_kernel on the K-quant bodies (q4k_gemv.h, q6k_gemv.h):
// two 8-wave workgroups per CU, each recording at most kKqFuseTiles tiles a
// wave in buffers that follow the body's LDS.  After the loop the slab rings
// are free: the last workgroup's loads, the histogram and the candidates go
// there.  All-greedy calls take it too (its greedy branch keeps each
// workgroup's packed maximum).
constexpr int kKqFuseTiles = 4;
template <int FMT>
size_t kq_sample_lds_bytes(int K) {
  return KqBody<FMT>::lds(K) + (size_t)KqBody<FMT>::kWaves * kKqFuseTiles * 16 * sizeof(uint2);
}
static_assert(KqBody<kW_Q6_K>::kRingBytes >= (size_t)kFuseMore * 4 + (size_t)kFuseStage * 12 &&
                  KqBody<kW_Q4_K>::kRingBytes >= (size_t)kFuseMore * 4 + (size_t)kFuseStage * 12,
              "the rings hold the waves read again and the candidates");

template <int FMT>
__global__ __launch_bounds__(KqBody<FMT>::kThreads, 2) void gemv_kq_sample_kernel(GemvArgs g, FuseArgs f) {
  constexpr int NW = KqBody<FMT>::kWaves;
  extern __shared__ uint4 qlds[];
  __shared__ FuseSmem fs;
  const int tid = threadIdx.x, wave = tid >> 6;
  const int m = (int)blockIdx.y;
  const bool rep = (load_scalar(&f.plans[m].pen) & kPenRep) != 0;
  float *y = g.y + (int64_t)m * g.ldy;

  // the row's repetition set: history.slice(-128), ids in [0, N)
  if (tid < kFuseSetSlots) fs.rset[tid] = -1;
  __syncthreads();
  if (rep) fuse_rep_set(f, m, g.N, fs.rset);
  // (the body's first barrier completes the set)

  uint8_t *lb = reinterpret_cast<uint8_t *>(qlds);
  uint2 *rec = reinterpret_cast<uint2 *>(lb + KqBody<FMT>::lds(g.K));
  RecordEpi epi{y, rec + wave * kKqFuseTiles * 16, rep ? fs.rset : nullptr, 0, kKqFuseTiles};
  KqBody<FMT>::run(g, lb, epi);
  int32_t *more = reinterpret_cast<int32_t *>(lb + KqBody<FMT>::ring_off(g.K));   // the rings
  fuse_sample_finish<NW>(g, f, m, epi.nt, kKqFuseTiles, rec, more,
                         reinterpret_cast<unsigned long long *>(more + kFuseMore), fs);
}

// Its grid: as the plain GEMV's (gemv_kq_mfma_kernel's launch); 0 when a
// wave would complete more than kKqFuseTiles tiles (its whole tiles and at
// most one part of a tail tile) or the last workgroup's threads would read
// more than kFuseWavesPerThread waves' entries.
template <int FMT>
int kq_sample_grid_t(const GemvArgs &g) {
  using B = KqBody<FMT>;
  const size_t lds = kq_sample_lds_bytes<FMT>(g.K);
  const int ntiles = (g.N + 15) / 16;
  const int res = resident_blocks(reinterpret_cast<const void *>(gemv_kq_sample_kernel<FMT>),
                                  (uint32_t)lds, B::kThreads);
  int blocks = (ntiles + B::kWaves - 1) / B::kWaves;
  blocks = blocks < res ? blocks : res;
  blocks = blocks < g.part_cap / B::kWaves ? blocks : g.part_cap / B::kWaves;
  if (blocks < 1 || !g.part || !g.tile_cnt) return 0;
  const int nw = blocks * B::kWaves;
  const int tiles = ntiles / nw + (ntiles % nw ? 1 : 0);
  return tiles <= kKqFuseTiles && nw <= kFuseWavesPerThread * B::kThreads ? blocks : 0;
}

int kq_sample_grid(const GemvArgs &g) {
  return g.type == kW_Q6_K   ? kq_sample_grid_t<kW_Q6_K>(g)
         : g.type == kW_Q4_K ? kq_sample_grid_t<kW_Q4_K>(g)
                             : 0;
}

int fuse_waves_per_block(int type) {
  return type == kW_Q6_K ? KqBody<kW_Q6_K>::kWaves : type == kW_Q4_K ? KqBody<kW_Q4_K>::kWaves : 16;
}
static_assert(tm::waves<kW_Q1_0>() == 16 && tm::waves<kW_PQ2_0>() == 16 &&
                  tm::waves<kW_PTQ1_0>() == 16,
              "fuse_waves_per_block: the planar kernels' waves");

template <int FMT>
hipError_t launch_kq_sample_t(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                              hipEvent_t *ev, hipEvent_t done) {
  const int blocks = kq_sample_grid_t<FMT>(g);
  if (blocks < 1 || blocks != f.blocks) return hipErrorInvalidValue;
  const size_t lds = kq_sample_lds_bytes<FMT>(g.K);
  const dim3 grid((unsigned)blocks, (unsigned)g.M), block(KqBody<FMT>::kThreads);
  if (ev)
    hipExtLaunchKernelGGL(gemv_kq_sample_kernel<FMT>, grid, block, lds, stream, ev[0], ev[1], 0u, g, f);
  else if (done)
    hipExtLaunchKernelGGL(gemv_kq_sample_kernel<FMT>, grid, block, lds, stream, nullptr, done, 0u, g, f);
  else
    hipLaunchKernelGGL(gemv_kq_sample_kernel<FMT>, grid, block, lds, stream, g, f);
  return hipGetLastError();
}

hipError_t launch_kq_sample(const GemvArgs &g, const FuseArgs &f, hipStream_t stream,
                            hipEvent_t *ev, hipEvent_t done) {
  switch (g.type) {
    case kW_Q6_K: return launch_kq_sample_t<kW_Q6_K>(g, f, stream, ev, done);
    case kW_Q4_K: return launch_kq_sample_t<kW_Q4_K>(g, f, stream, ev, done);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------- launch

hipError_t prepare_kernels() {
  hipError_t e0 = prepare_gemv();
  if (e0 != hipSuccess) return e0;
  const int pen_smem = (int)pen_smem_bytes();
  const int row_smem = (int)row_smem_bytes(kRowMaxVocab);
  hipError_t e;
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&pen_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, pen_smem)) != hipSuccess)
    return e;
  const void *row_k[4] = {reinterpret_cast<const void *>(&row_kernel<true, false>),
                          reinterpret_cast<const void *>(&row_kernel<false, false>),
                          reinterpret_cast<const void *>(&row_kernel<true, true>),
                          reinterpret_cast<const void *>(&row_kernel<false, true>)};
  for (const void *f : row_k)
    if ((e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, row_smem)) !=
        hipSuccess)
      return e;
  const int mid_smem = kMidLdsMax;
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&mid_kernel<true>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, mid_smem)) != hipSuccess)
    return e;
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&mid_kernel<false>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, mid_smem)) != hipSuccess)
    return e;
  {
    const void *tk[3] = {reinterpret_cast<const void *>(&gemv_tern_sample_kernel<kW_Q1_0>),
                         reinterpret_cast<const void *>(&gemv_tern_sample_kernel<kW_PQ2_0>),
                         reinterpret_cast<const void *>(&gemv_tern_sample_kernel<kW_PTQ1_0>)};
    for (const void *fk : tk)
      if ((e = hipFuncSetAttribute(fk, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)tern_sample_lds_bytes(kGemvMaxK, 16))) != hipSuccess)
        return e;
    const void *kk[4] = {reinterpret_cast<const void *>(&gemv_kq_sample_kernel<kW_Q6_K>),
                         reinterpret_cast<const void *>(&gemv_kq_sample_kernel<kW_Q4_K>),
                         reinterpret_cast<const void *>(&gemv_kq_argmax_kernel<kW_Q6_K>),
                         reinterpret_cast<const void *>(&gemv_kq_argmax_kernel<kW_Q4_K>)};
    const size_t kl[4] = {kq_sample_lds_bytes<kW_Q6_K>(kGemvMaxK), kq_sample_lds_bytes<kW_Q4_K>(kGemvMaxK),
                          KqBody<kW_Q6_K>::lds(kGemvMaxK), KqBody<kW_Q4_K>::lds(kGemvMaxK)};
    for (int i = 0; i < 4; ++i)
      if ((e = hipFuncSetAttribute(kk[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)kl[i])) !=
          hipSuccess)
        return e;
    const void *ak[3] = {reinterpret_cast<const void *>(&gemv_tern_argmax_kernel<kW_Q1_0>),
                         reinterpret_cast<const void *>(&gemv_tern_argmax_kernel<kW_PQ2_0>),
                         reinterpret_cast<const void *>(&gemv_tern_argmax_kernel<kW_PTQ1_0>)};
    for (const void *fk : ak)
      if ((e = hipFuncSetAttribute(fk, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)gemv_tern_lds_bytes(kGemvMaxK))) != hipSuccess)
        return e;
  }
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&finalize_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)finalize_smem_bytes())) != hipSuccess)
    return e;
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&large_fast_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)large_fast_smem_bytes())) != hipSuccess)
    return e;
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&large_replay_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)replay_smem_bytes())) != hipSuccess)
    return e;
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void *>(&large_replay_dev_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)replay_dev_smem_bytes())) != hipSuccess)
    return e;
  return hipFuncSetAttribute(reinterpret_cast<const void *>(&large_kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)large_smem_bytes());
}

namespace {

// One launch; with events, hipExtLaunchKernelGGL stamps the start and end of
// the kernel's own dispatch (no marker packets are added to the stream).
// Without them, `done` (when not null) is recorded at the kernel's end the
// same way.
template <typename K>
hipError_t launch_one(K kernel, dim3 grid, dim3 block, size_t smem, hipStream_t stream,
                      hipEvent_t *ev, int slot, hipEvent_t done, const LaunchArgs &a,
                      const Workspace &ws) {
  if (ev)
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)smem, stream, ev[2 * slot],
                          ev[2 * slot + 1], 0u, a, ws);
  else if (done)
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)smem, stream, nullptr, done, 0u, a,
                          ws);
  else
    hipLaunchKernelGGL(kernel, grid, block, smem, stream, a, ws);
  return hipGetLastError();
}

}  // namespace

// A decode step's bookkeeping as a kernel of its own (put_token's, one
// thread per row), for the calls whose tokens no sampler kernel writes (an
// empty vocabulary: every token 0).
__global__ __launch_bounds__(256) void decode_append_kernel(DecodeArgs d) {
  const int r = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (r >= d.rows) return;
  // every read first (one round trip), then the decision and the writes
  const int done = d.done[r];
  const int t = d.tokens[r];
  int64_t len = d.len[r];
  bool stop = false;
  for (int i = 0; i < d.n_stop; ++i) stop |= d.stop_ids[i] == t;
  if (done != 0) {
    d.tokens[r] = -1;
    return;
  }
  if (stop) {
    d.done[r] = 1;
    return;
  }
  if (len < 0) len = 0;
  d.ring[(int64_t)r * d.cap + len % d.cap] = t;
  d.len[r] = len + 1;
}

// What a host call copies back, written straight into its pinned buffer:
// dst[i] = src[idx[i]] for i < n (the penalised logits; idx is read from the
// pinned buffer too) and tok_dst[r] = tok[r] for r < rows.
__global__ __launch_bounds__(256) void gather_out_kernel(const float *src, const int64_t *idx,
                                                         float *dst, int64_t n, const int32_t *tok,
                                                         int32_t *tok_dst, int32_t rows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[idx[i]];
  else if (i < n + rows) tok_dst[i - n] = tok[i - n];
}

hipError_t launch_gather_out(const float *src, const int64_t *idx, float *dst, int64_t n,
                             const int32_t *tok, int32_t *tok_dst, int32_t rows,
                             hipStream_t stream) {
  const int64_t total = n + rows;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_out_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                     src, idx, dst, n, tok, tok_dst, rows);
  return hipGetLastError();
}

// Sets n words to v: a kernel, not hipMemsetAsync, so that a caller may
// capture it in a graph.
__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t *p, int64_t n, uint32_t v, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p,
                     n, v);
  return hipGetLastError();
}

hipError_t launch_decode_append(const DecodeArgs &d, hipStream_t stream) {
  if (d.rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(decode_append_kernel, dim3((unsigned)((d.rows + 255) / 256)), dim3(256), 0,
                     stream, d);
  return hipGetLastError();
}

hipError_t launch_sample(const LaunchArgs &a, const Workspace &ws, hipStream_t stream,
                         hipEvent_t *ev, hipEvent_t done) {
  hipError_t e;
  // the last kernel of the call records `done`
  const int last = a.n_argmax > 0 ? 6 : a.n_large > 0 && a.replay_dev > 0 ? 10
                 : a.n_large > 0 ? 9 : a.n_lfast > 0 ? 4
                 : a.n_chunk > 0 ? 3 : a.n_mid > 0 ? 5 : a.n_row > 0 ? 1 : 0;
  auto dn = [&](int slot) { return slot == last ? done : nullptr; };
  if (a.n_pf > 0) {
    e = launch_one(pen_kernel, dim3((unsigned)a.n_pf), dim3(kPenThreads), pen_smem_bytes(),
                   stream, ev, 0, dn(0), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_row > 0) {
    const size_t smem = row_smem_bytes(a.vocab);
    if (a.split > 1) {
      const dim3 grid((unsigned)(a.n_row * a.split));
      e = a.vec ? launch_one(row_kernel<true, true>, grid, dim3(kRowThreads), smem, stream, ev, 1, dn(1), a, ws)
                : launch_one(row_kernel<false, true>, grid, dim3(kRowThreads), smem, stream, ev, 1, dn(1), a, ws);
    } else {
      const dim3 grid((unsigned)a.n_row);
      e = a.vec ? launch_one(row_kernel<true, false>, grid, dim3(kRowThreads), smem, stream, ev, 1, dn(1), a, ws)
                : launch_one(row_kernel<false, false>, grid, dim3(kRowThreads), smem, stream, ev, 1, dn(1), a, ws);
    }
    if (e != hipSuccess) return e;
  }
  if (a.n_mid > 0) {
    const size_t smem = mid_smem_bytes(a.vocab);
    e = a.vec ? launch_one(mid_kernel<true>, dim3((unsigned)a.n_mid), dim3(kRowThreads), smem,
                           stream, ev, 5, dn(5), a, ws)
              : launch_one(mid_kernel<false>, dim3((unsigned)a.n_mid), dim3(kRowThreads), smem,
                           stream, ev, 5, dn(5), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_chunk > 0) {
    const dim3 grid((unsigned)(a.n_chunk * a.chunks));
    e = a.vec ? launch_one(chunk_kernel<true>, grid, dim3(kThreads), 0, stream, ev, 2, dn(2), a, ws)
              : launch_one(chunk_kernel<false>, grid, dim3(kThreads), 0, stream, ev, 2, dn(2), a, ws);
    if (e != hipSuccess) return e;
    e = launch_one(finalize_kernel, dim3((unsigned)a.n_chunk), dim3(kThreads),
                   finalize_smem_bytes(), stream, ev, 3, dn(3), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_lfast > 0) {
    e = launch_one(large_fast_kernel, dim3((unsigned)a.n_lfast), dim3(kFT), large_fast_smem_bytes(),
                   stream, ev, 8, dn(8), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_large + a.n_lfast > 0) {
    e = launch_one(large_kernel, dim3((unsigned)(a.n_large + a.n_lfast)), dim3(kLT),
                   large_smem_bytes(), stream, ev, 4, dn(4), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_large > 0) {   // rows of large_list that asked for the slot replay
    e = launch_one(large_replay_kernel, dim3((unsigned)a.n_large), dim3(kLT), replay_smem_bytes(),
                   stream, ev, 9, dn(9), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_large > 0 && a.replay_dev > 0) {   // the replays whose slots live in device memory
    e = launch_one(large_replay_dev_kernel, dim3((unsigned)a.replay_dev), dim3(kLT),
                   replay_dev_smem_bytes(), stream, ev, 10, dn(10), a, ws);
    if (e != hipSuccess) return e;
  }
  if (a.n_argmax > 0) {
    const dim3 grid((unsigned)(a.n_argmax * a.split));
    e = a.vec ? launch_one(argmax_kernel<true>, grid, dim3(kRowThreads), 0, stream, ev, 6, dn(6), a, ws)
              : launch_one(argmax_kernel<false>, grid, dim3(kRowThreads), 0, stream, ev, 6, dn(6), a, ws);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace hs
