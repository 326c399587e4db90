// gfx950 kernels of the logits-to-token sampler.
//
// Semantics follow hachiue's sampleLogits (src/sampler.ts:12-118): logits are
// binary32, all arithmetic after the load is binary64 and results are rounded
// to binary32 exactly where the reference stores into a Float32Array.  This
// file must be compiled with -ffp-contract=off so no multiply-add is fused.
//
// Pipeline per call (two launches):
//   chunk_kernel     grid rows*S, 256 threads.  Each workgroup owns 16384
//                    consecutive logits of one row, held in registers (one
//                    HBM read).  It applies the penalties in place, then:
//                    greedy rows  -> (max, first index) of the chunk;
//                    k <= 64      -> every logit >= X_c, where X_c is the
//                                    largest per-wave "k-th largest lane
//                                    maximum" (a lower bound of the chunk's
//                                    k-th largest value);
//                    k <= 1024    -> every logit >= the chunk's exact k-th
//                                    largest value (workgroup radix select).
//                    Candidates are appended to one contiguous list per row.
//   finalize_kernel  grid rows, 256 threads.  Exact k-th largest over the
//                    row's candidates, stable descending order, tie
//                    detection with an exact replace-min replay when a tie
//                    can change the result, then the binary64 softmax,
//                    min-p / top-p cutoff and the draw.
#include "sampler_internal.h"

#include <math.h>

#include "hachiue_sampler.h"

namespace hs {

// ---------------------------------------------------------------- helpers

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Order-preserving key of a binary32 value: larger value <=> larger key.
// NaN and -Infinity (which never enter the reference's top-k, since
// `v > minVal` is false for them, src/sampler.ts:57) map to 0.
__device__ __forceinline__ uint32_t f2key(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (f > -INFINITY) ? k : 0u;
}

__device__ __forceinline__ float key2f(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

// Candidate composite: key in the high word, ~index in the low word, so a
// descending sort orders by value descending and index ascending.
__device__ __forceinline__ unsigned long long pack_cand(uint32_t key, uint32_t idx) {
  return ((unsigned long long)key << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t cand_key(unsigned long long c) { return (uint32_t)(c >> 32); }
__device__ __forceinline__ uint32_t cand_idx(unsigned long long c) { return 0xFFFFFFFFu - (uint32_t)c; }

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

__device__ __forceinline__ uint32_t lanes_below(unsigned long long mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Bitonic sort of one value per lane across a wave64, descending.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t x) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t y = __shfl_xor(x, stride);
      const bool lower = (lane & stride) == 0;
      const bool desc = (lane & size) == 0;
      x = (lower == desc) ? max(x, y) : min(x, y);
    }
  }
  return x;
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

// Inclusive prefix sum over the 256 threads of the block.  `wsum` is 4 words
// of shared memory.  Contains one barrier; callers separate reuses of wsum by
// at least one more barrier.
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

// Scratch of the block radix select.
struct SelectSmem {
  uint32_t hist[256];
  uint32_t wsum[4];
  int32_t digit, above, total;
};

// k-th largest key of a block-wide multiset, four 8-bit digit passes over a
// shared 256-bin histogram.  `hist_pass(shift, prefix, pass)` adds this
// thread's participating keys (keys equal to 0 never participate) whose
// digits above `shift` equal `prefix`'s.  Returns the exact key T, or 0 when
// fewer than k keys participate; *total receives the participant count.
template <typename HistPass>
__device__ uint32_t block_select_core(int k, HistPass hist_pass, SelectSmem &sm, int *total) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0;
  int rem = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    sm.hist[tid] = 0;
    __syncthreads();
    hist_pass(shift, prefix, pass);
    __syncthreads();
    const uint32_t c = sm.hist[255 - tid];
    const uint32_t incl = block_scan_incl(c, sm.wsum);
    if (pass == 0 && tid == 255) sm.total = (int)incl;
    if (incl >= (uint32_t)rem && incl - c < (uint32_t)rem) {
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

__device__ __forceinline__ void hist_add(SelectSmem &sm, uint32_t key, int shift, uint32_t prefix,
                                         int pass) {
  if (key == 0) return;
  if (pass > 0 && (key >> (shift + 8)) != (prefix >> (shift + 8))) return;
  atomicAdd(&sm.hist[(key >> shift) & 255u], 1u);
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

// ---------------------------------------------------------------- chunk kernel

template <bool VEC>
__global__ __launch_bounds__(kThreads) void chunk_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ uint32_t dyn[];   // touched bits | repetition bits | counts
  __shared__ SelectSmem sel;
  __shared__ unsigned long long s_best[kWaves];
  __shared__ uint32_t s_thr[kWaves];
  __shared__ int32_t s_cnt, s_base, s_over;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = a.chunks;
  const int row = blockIdx.x / S;
  const int chunk = blockIdx.x - row * S;
  const RowPlan P = ws.plans[row];
  float *rowp = a.logits + (int64_t)row * a.stride;
  const int lo = chunk * kChunk;
  const int hi = min(lo + kChunk, a.vocab);
  const int wbase = lo + wave * kWaveSpan;

  // 1. one HBM read of the chunk into registers (coalesced float4 per lane)
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

  // 2. penalties on the ids of this chunk, applied in registers and written
  //    back in place (the reference mutates the caller's logits).
  if (P.pen) {
    uint32_t *touched = dyn;
    uint32_t *repbits = dyn + kChunk / 32;
    uint32_t *counts = dyn + 2 * (kChunk / 32);
    for (int i = tid; i < kChunk / 32; i += kThreads) { touched[i] = 0; repbits[i] = 0; }
    if (P.pen & kPenPF)
      for (int i = tid; i < kChunk; i += kThreads) counts[i] = 0;
    __syncthreads();
    const int64_t h0 = a.hist_off ? a.hist_off[row] : 0;
    const int64_t hl = a.hist_off ? a.hist_off[row + 1] - h0 : 0;
    if (P.pen & kPenRep) {
      const int64_t last = hl < 128 ? hl : 128;   // history.slice(-128)
      for (int64_t t = tid; t < last; t += kThreads) {
        const int id = a.hist_ids[h0 + hl - last + t];
        if (id >= lo && id < hi) {
          const int o = id - lo;
          atomicOr(&touched[o >> 5], 1u << (o & 31));
          atomicOr(&repbits[o >> 5], 1u << (o & 31));
        }
      }
    }
    if (P.pen & kPenPF) {
      for (int64_t t = tid; t < hl; t += kThreads) {
        const int id = a.hist_ids[h0 + t];
        if (id >= lo && id < hi) {
          const int o = id - lo;
          atomicAdd(&counts[o], 1u);
          atomicOr(&touched[o >> 5], 1u << (o & 31));
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kNV; ++j) {
      const int e = wbase + (j * 64 + lane) * 4;
      if (e >= hi) continue;
      const int o = e - lo;
      const uint32_t bits = (touched[o >> 5] >> (o & 31)) & 0xFu;
      if (bits) {
        const uint32_t rb = (repbits[o >> 5] >> (o & 31)) & 0xFu;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (bits & (1u << q)) {
            const uint32_t n = (P.pen & kPenPF) ? counts[o + q] : 0u;
            const float nv = penalise(v[j][q], (rb >> q) & 1u, n, P);
            v[j][q] = nv;
            rowp[e + q] = nv;
          }
        }
      }
    }
  }

  ChunkInfo *info = ws.info + (int64_t)row * S + chunk;
  uint2 *rowcand = ws.cand + (int64_t)row * ((int64_t)S * kChunkCap);
  const int cap = S * kChunkCap;

  if (P.mode == kModeGreedy) {
    // src/sampler.ts:37-45: first index of the maximum (NaN never wins).
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

  if (P.mode == kModeSmall) {
    // Lower bound of the chunk's k-th largest value: the k-th largest lane
    // maximum of a wave is <= that wave's k-th largest logit.
    const int k = P.k;
    float lm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kNV; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) lm = fmaxf(lm, v[j][q]);
    const uint32_t sorted = wave_sort_desc(f2key(lm));
    const uint32_t mw = __shfl(sorted, k - 1);
    if (lane == 0) s_thr[wave] = mw;
    if (tid == 0) { s_over = 0; }
    __syncthreads();
    uint32_t X = max(max(s_thr[0], s_thr[1]), max(s_thr[2], s_thr[3]));
    if (X == 0) X = 1;   // fewer than k finite lane maxima: keep every finite logit

    // count, reserve, write (ballot compaction; almost every ballot is empty)
    uint32_t cnt = 0;
#pragma unroll
    for (int j = 0; j < kNV; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) cnt += (uint32_t)__popcll(__ballot(f2key(v[j][q]) >= X));
    int base = 0;
    if (lane == 0 && cnt) base = atomicAdd(&ws.cand_count[row], (int)cnt);
    base = __shfl(base, 0);
    if (base + (int)cnt > cap && lane == 0) atomicOr(&s_over, 1);
    uint32_t pos = 0;
#pragma unroll
    for (int j = 0; j < kNV; ++j) {
      const int e = wbase + (j * 64 + lane) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t key = f2key(v[j][q]);
        const bool pass = key >= X;
        const unsigned long long b = __ballot(pass);
        if (b) {
          const int p = base + (int)(pos + lanes_below(b));
          if (pass && p < cap) rowcand[p] = make_uint2(key, (uint32_t)(e + q));
          pos += (uint32_t)__popcll(b);
        }
      }
    }
    if (lane == 0) s_thr[wave] = cnt;   // reuse: per-wave counts for the finite total
    __syncthreads();
    if (tid == 0) {
      info->best = 0;
      info->thr = X;
      info->overflow = s_over;
      // With X == 1 every finite logit was kept, so the count is exact.
      info->finite = (X == 1 && !s_over) ? (int)(s_thr[0] + s_thr[1] + s_thr[2] + s_thr[3]) : -1;
    }
    return;
  }

  if (P.mode == kModeGeneric) {
    const int k = P.k;
    int total = 0;
    const uint32_t T = block_select_core(
        k,
        [&](int shift, uint32_t prefix, int pass) {
#pragma unroll
          for (int j = 0; j < kNV; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) hist_add(sel, f2key(v[j][q]), shift, prefix, pass);
        },
        sel, &total);
    const uint32_t X = T ? T : 1u;   // fewer than k finite: keep them all
    if (tid == 0) { s_cnt = 0; s_over = 0; }
    __syncthreads();
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < kNV; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) mine += f2key(v[j][q]) >= X ? 1u : 0u;
    const uint32_t off = block_scan_incl(mine, sel.wsum) - mine;
    if (tid == kThreads - 1) s_cnt = (int)(off + mine);
    __syncthreads();
    if (tid == 0) {
      s_base = s_cnt ? atomicAdd(&ws.cand_count[row], s_cnt) : 0;
      if (s_base + s_cnt > cap) s_over = 1;
    }
    __syncthreads();
    int p = s_base + (int)off;
#pragma unroll
    for (int j = 0; j < kNV; ++j) {
      const int e = wbase + (j * 64 + lane) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t key = f2key(v[j][q]);
        if (key >= X) {
          if (p < cap) rowcand[p] = make_uint2(key, (uint32_t)(e + q));
          ++p;
        }
      }
    }
    if (tid == 0) {
      info->best = 0;
      info->thr = X;
      info->overflow = s_over;
      info->finite = total;
    }
    return;
  }
}

// ---------------------------------------------------------------- finalize

struct FinalSmem {
  SelectSmem sel;
  unsigned long long red[kWaves];
  uint32_t xrow;
  int32_t finite_sum, finite_known, overflow, n_all, n_sel;
  int32_t n, token, cutoff, pick, replay;
  double sum, kept;
};

// Exact replace-min scan of src/sampler.ts:50-69 over the whole (already
// penalised) row by wave 0: slot j holds (sv[j], sid[j]); a logit enters iff
// it is strictly greater than the current minimum, into the first slot
// holding that minimum.  Logits are consumed in index order.
__device__ void replay_row(const float *rowp, int vocab, int k, float *sv, int32_t *sid) {
  const int lane = lane_id();
  for (int j = lane; j < k; j += 64) { sv[j] = -INFINITY; sid[j] = -1; }
  float mv = -INFINITY;
  int mi = 0;
  constexpr int kBlk = 16;   // 1024 logits per step, loads issued together
  for (int base = 0; base < vocab; base += 64 * kBlk) {
    float x[kBlk];
#pragma unroll
    for (int q = 0; q < kBlk; ++q) {
      const int e = base + q * 64 + lane;
      x[q] = e < vocab ? rowp[e] : __builtin_nanf("");
    }
#pragma unroll
    for (int q = 0; q < kBlk; ++q) {
      int done = -1;
      for (;;) {
        const unsigned long long b = __ballot(x[q] > mv && lane > done);
        if (!b) break;
        const int L = __ffsll((long long)b) - 1;
        const float vL = __shfl(x[q], L);
        // a wave's LDS accesses complete in program order, so every lane's
        // rescan below observes this store
        if (lane == 0) { sv[mi] = vL; sid[mi] = base + q * 64 + L; }
        // rescan: first slot with the minimum value (strict '<' from slot 0)
        float bv = INFINITY;
        int bj = 0x7FFFFFFF;
        for (int j = lane; j < k; j += 64) {
          const float s = sv[j];
          if (bj == 0x7FFFFFFF || s < bv) { bv = s; bj = j; }
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
        mi = bj;
        done = L;
      }
    }
  }
}

// Bitonic sort of P (power of two) packed candidates in shared memory,
// descending.  All threads of the block participate.
__device__ void block_sort_desc(unsigned long long *a, int P) {
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P / 2; i += kThreads) {
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

__global__ __launch_bounds__(kThreads) void finalize_kernel(LaunchArgs a, Workspace ws) {
  extern __shared__ unsigned long long fdyn[];
  unsigned long long *ent = fdyn;                    // kFinalCap
  unsigned long long *sorted = fdyn + kFinalCap;     // 2048
  uint32_t *skey = reinterpret_cast<uint32_t *>(sorted + 2048);   // kMaxK
  int32_t *sids = reinterpret_cast<int32_t *>(skey + kMaxK);      // kMaxK
  float *sprob = reinterpret_cast<float *>(sids + kMaxK);          // kMaxK
  double *sp = reinterpret_cast<double *>(sprob + kMaxK);          // kMaxK
  float *rsv = reinterpret_cast<float *>(sp + kMaxK);              // kMaxK
  int32_t *rsid = reinterpret_cast<int32_t *>(rsv + kMaxK);        // kMaxK
  __shared__ FinalSmem f;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.x;
  const int S = a.chunks;
  const RowPlan P = ws.plans[row];
  const float *rowp = a.logits + (int64_t)row * a.stride;
  const ChunkInfo *info = ws.info + (int64_t)row * S;
  const int cs = a.cand_stride;

  if (P.mode == kModeGreedy) {
    unsigned long long best = 0;
    for (int c = tid; c < S; c += kThreads) best = info[c].best > best ? info[c].best : best;
    best = wave_max64(best);
    if (lane == 0) f.red[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = f.red[0];
      for (int w = 1; w < kWaves; ++w) b = f.red[w] > b ? f.red[w] : b;
      int token = b ? (int)cand_idx(b) : 0;
      if (isnan(rowp[0])) token = 0;   // bestVal = logits[0] = NaN: nothing is '>' it
      a.tokens[row] = token;
      if (a.cand_count_out) a.cand_count_out[row] = 0;
      if (a.cutoff_out) a.cutoff_out[row] = 0;
      if (a.row_flags) a.row_flags[row] = HS_ROW_GREEDY;
    }
    return;
  }

  const int k = P.k;

  // ---- row summary
  if (tid == 0) {
    f.xrow = 0; f.finite_sum = 0; f.finite_known = 1; f.overflow = 0; f.n_all = 0;
    f.replay = 0;
  }
  __syncthreads();
  for (int c = tid; c < S; c += kThreads) {
    atomicMax(&f.xrow, info[c].thr);
    if (info[c].overflow) atomicOr(&f.overflow, 1);
    if (info[c].finite < 0) atomicAnd(&f.finite_known, 0);
    else atomicAdd(&f.finite_sum, info[c].finite);
  }
  __syncthreads();
  const int n_rowcand = min(ws.cand_count[row], S * kChunkCap);
  const uint2 *rowcand = ws.cand + (int64_t)row * ((int64_t)S * kChunkCap);
  const uint32_t xrow = f.xrow;
  bool closed_form = f.finite_known && f.finite_sum <= k && !f.overflow;
  bool need_replay = f.overflow;

  // ---- gather candidates >= X_row into shared memory
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
  const int n_all = min(f.n_all, kFinalCap);

  int n = 0;
  bool boundary_tie = false, internal_tie = false;
  uint32_t T = 0;
  if (!need_replay) {
    int total = 0;
    if (n_all > k) {
      T = block_select_core(
          k,
          [&](int shift, uint32_t prefix, int pass) {
            for (int p = tid; p < n_all; p += kThreads)
              hist_add(f.sel, cand_key(ent[p]), shift, prefix, pass);
          },
          f.sel, &total);
    }
    // entries >= T (all entries when n_all <= k)
    if (tid == 0) f.n_sel = 0;
    __syncthreads();
    for (int i = tid; i < n_all; i += kThreads) {
      const unsigned long long c = ent[i];
      if (cand_key(c) >= T) {
        const int p = atomicAdd(&f.n_sel, 1);
        if (p < 2048) sorted[p] = c;
      }
    }
    __syncthreads();
    const int n_sel = f.n_sel;
    if (n_sel > 2048) {
      need_replay = true;
    } else {
      int P2 = 1;
      while (P2 < n_sel) P2 <<= 1;
      for (int i = n_sel + tid; i < P2; i += kThreads) sorted[i] = 0ull;
      __syncthreads();
      if (P2 <= 64) {
        if (wave == 0) {
          unsigned long long x = lane < P2 ? sorted[lane] : 0ull;
          x = wave_sort_desc64(x);
          if (lane < P2) sorted[lane] = x;
        }
        __syncthreads();
      } else {
        block_sort_desc(sorted, P2);
      }
      n = n_sel < k ? n_sel : k;
      boundary_tie = n_sel > k;
      for (int i = tid; i < n; i += kThreads) {
        skey[i] = cand_key(sorted[i]);
        sids[i] = (int32_t)cand_idx(sorted[i]);
      }
      __syncthreads();
      // equal neighbours inside the kept candidates
      int tie = 0;
      for (int i = tid; i + 1 < n; i += kThreads) tie |= skey[i] == skey[i + 1];
      internal_tie = __syncthreads_or(tie) != 0;
      if (closed_form) { boundary_tie = false; internal_tie = false; }
      // exact membership / order needed for the candidate outputs
      if ((boundary_tie || internal_tie) && a.want_cands) need_replay = true;
    }
  }

  // ---- tail (binary64), src/sampler.ts:76-117; may run twice if a tie
  //      group holds the drawn position and the order must be replayed.
  const double u = a.uniforms[row];
  for (int attempt = 0; attempt < 2; ++attempt) {
    if (need_replay) {
      if (wave == 0) replay_row(rowp, a.vocab, k, rsv, rsid);
      __syncthreads();
      if (tid == 0) f.n_sel = 0;
      __syncthreads();
      for (int j = tid; j < k; j += kThreads) {
        if (rsid[j] >= 0) {
          const int p = atomicAdd(&f.n_sel, 1);
          sorted[p] = pack_cand(f2key(rsv[j]), (uint32_t)j);
        }
      }
      __syncthreads();
      const int n_sel = f.n_sel;
      int P2 = 1;
      while (P2 < n_sel) P2 <<= 1;
      for (int i = n_sel + tid; i < P2; i += kThreads) sorted[i] = 0ull;
      __syncthreads();
      block_sort_desc(sorted, P2);
      n = n_sel;
      for (int i = tid; i < n; i += kThreads) {
        const uint32_t slot = cand_idx(sorted[i]);
        skey[i] = cand_key(sorted[i]);
        sids[i] = rsid[slot];
      }
      if (tid == 0) f.replay = 1;
      __syncthreads();
      boundary_tie = internal_tie = false;
    }

    if (n >= 2) {
      const double maxl = (double)key2f(skey[0]);
      const double inv_temp = 1.0 / P.temperature;
      for (int i = tid; i < n; i += kThreads) {
        const double p = exp(((double)key2f(skey[i]) - maxl) * inv_temp);
        sp[i] = p;
        sprob[i] = (float)p;
      }
      __syncthreads();
      if (tid == 0) {
        double s = 0;
        for (int i = 0; i < n; ++i) s += sp[i];
        f.sum = s;
      }
      __syncthreads();
      const double s = f.sum;
      for (int i = tid; i < n; i += kThreads) sprob[i] = (float)((double)sprob[i] / s);
      __syncthreads();
      if (tid == 0) {
        const double thr = P.min_p * (double)sprob[0];
        double cum = 0;
        int cut = n;
        for (int i = 0; i < n; ++i) {
          if (i > 0 && (double)sprob[i] < thr) { cut = i; break; }
          cum += (double)sprob[i];
          if (cum >= P.top_p) { cut = i + 1; break; }
        }
        double kept = 0;
        for (int i = 0; i < cut; ++i) kept += (double)sprob[i];
        double r = u * kept;
        int pick = cut - 1;
        for (int i = 0; i < cut; ++i) {
          r -= (double)sprob[i];
          if (r <= 0) { pick = i; break; }
        }
        f.cutoff = cut;
        f.pick = pick;
      }
      __syncthreads();
    } else {
      if (tid == 0) { f.cutoff = n; f.pick = n == 1 ? 0 : -1; }
      __syncthreads();
    }

    if (attempt == 0 && !need_replay && (boundary_tie || internal_tie)) {
      // The order inside a group of equal values depends on the slot
      // history; it matters only if the drawn position is inside one.
      const int pick = f.pick;
      bool hit = false;
      if (pick >= 0) {
        const uint32_t kp = skey[pick];
        hit = (pick > 0 && skey[pick - 1] == kp) || (pick + 1 < n && skey[pick + 1] == kp) ||
              (boundary_tie && kp == T);
      }
      if (hit) { need_replay = true; continue; }
    }
    break;
  }

  if (tid == 0) {
    const int pick = f.pick;
    a.tokens[row] = pick >= 0 ? sids[pick] : 0;
    if (a.cand_count_out) a.cand_count_out[row] = n;
    if (a.cutoff_out) a.cutoff_out[row] = f.cutoff;
    if (a.row_flags) {
      uint32_t fl = 0;
      if (f.replay) fl |= HS_ROW_REPLAYED;
      if (boundary_tie || internal_tie || f.replay) fl |= HS_ROW_TIES;
      if (n < 2) fl |= HS_ROW_SINGLE;
      a.row_flags[row] = fl;
    }
    ws.cand_count[row] = 0;   // ready for the next call on this workspace
  }
  if (a.cand_ids || a.cand_probs) {
    for (int i = tid; i < n && i < cs; i += kThreads) {
      if (a.cand_ids) a.cand_ids[(int64_t)row * cs + i] = sids[i];
      if (a.cand_probs) a.cand_probs[(int64_t)row * cs + i] = n >= 2 ? sprob[i] : 1.0f;
    }
  }
}

size_t finalize_smem_bytes() {
  return (size_t)kFinalCap * 8 + 2048 * 8 + (size_t)kMaxK * (4 + 4 + 4 + 8 + 4 + 4);
}

hipError_t prepare_kernels() {
  const int chunk_max = (2 * (kChunk / 32) + kChunk) * 4;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&chunk_kernel<true>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, chunk_max);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute(reinterpret_cast<const void *>(&chunk_kernel<false>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, chunk_max);
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute(reinterpret_cast<const void *>(&finalize_kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)finalize_smem_bytes());
}

hipError_t launch_sample(const LaunchArgs &a, const Workspace &ws, hipStream_t stream,
                         hipEvent_t *ev) {
  const size_t chunk_smem = (size_t)(2 * (kChunk / 32) + (a.any_pf ? kChunk : 0)) * 4;
  const dim3 grid((unsigned)(a.rows * a.chunks));
  hipError_t e;
  if (ev && (e = hipEventRecord(ev[0], stream)) != hipSuccess) return e;
  if (a.vec)
    hipLaunchKernelGGL(chunk_kernel<true>, grid, dim3(kThreads), chunk_smem, stream, a, ws);
  else
    hipLaunchKernelGGL(chunk_kernel<false>, grid, dim3(kThreads), chunk_smem, stream, a, ws);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[1], stream)) != hipSuccess) return e;
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)a.rows), dim3(kThreads),
                     finalize_smem_bytes(), stream, a, ws);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[2], stream)) != hipSuccess) return e;
  return hipSuccess;
}

}  // namespace hs
