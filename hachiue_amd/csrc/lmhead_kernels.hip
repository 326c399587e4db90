// gfx950 lm_head GEMV: the logits producer in front of the sampler.
//
// hachiue's forward pass ends in output.weight [N = vocab rows x K] times the
// final normalised hidden state (src/engine.ts:1493-1515), dispatched to one
// of its WGSL GEMV pipelines by weight type (src/engine.ts:1156-1183,
// src/kernels.ts:244-290, :717-1090).  The weight tensor is the GGUF tensor's
// raw blocks, rows back to back (src/engine.ts:772-800); these kernels read it
// in place: F32, Q4_0 (18 B / 32 weights), Q4_1 (20 B / 32), Q4_K (144 B /
// 256), Q6_K (210 B / 256).
//
// Q4_K and Q6_K run on the matrix cores (gemv_kq_mfma_kernel; the bodies in
// q4k_gemv.h and q6k_gemv.h).  F32, Q4_0 and Q4_1 use the vector units, one
// wave per group of rows:
//   every lane owns a fixed "unit" of each row: 32 weights.  Its slice of x
//   stays in registers
//   for every row, with the sums the formats' offsets need (sum x over a
//   group).  A row takes `seg` lanes (the row's units rounded up to a power of
//   two; 64 / seg rows per wave step), or all 64 lanes with two units each.
//   The lanes of a row add their partial sums by DPP moves and the last
//   writes y.  Weights are read once, through a buffer resource: F32 in
//   aligned 16-byte loads, the block formats through LDS (gemv_lds_kernel).
// Quant nibbles become floats a byte at a time (v_cvt_f32_ubyte*), four per
// dword, and enter binary32 fused multiply-adds; the result differs from the
// reference's binary32 sums by rounding only (its own order is not a
// specification: WGSL leaves contraction and evaluation to the compiler).
#include "sampler_internal.h"
#include "blk_gemv.h"
#include "kq_gemv.h"
#include "tern_gemv.h"

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

namespace hs {


// ---- F32, Q4_0, Q4_1 on the vector units (the bodies: blk_gemv.h)

namespace {
// Each row's (or tile's) results straight to y.
struct StoreRow {
  float *y;
  __device__ __forceinline__ void out(int, int row, float v, bool valid) {
    if (valid) y[row] = v;
  }
};
}  // namespace

template <int FMT, int NRU>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs g) {
  StoreRow epi{g.y + (int64_t)blockIdx.y * g.ldy};
  gemv_vec_body<FMT, NRU>(g, epi);
}

template <int FMT, int NRU>
__global__ __launch_bounds__(kGemvThreads) void gemv_lds_kernel(GemvArgs g) {
  extern __shared__ uint4 glds[];
  StoreRow epi{g.y + (int64_t)blockIdx.y * g.ldy};
  gemv_lds_body<FMT, NRU>(g, glds, epi);
}

// ---- Q4_K and Q6_K on the matrix cores (the bodies: q4k_gemv.h, q6k_gemv.h)

// 2 workgroups per CU (16 waves): at most 128 VGPRs
template <int FMT>
__global__ __launch_bounds__(KqBody<FMT>::kThreads, 2) void gemv_kq_mfma_kernel(GemvArgs g) {
  extern __shared__ uint4 qlds[];
  StoreRow epi{g.y + (int64_t)blockIdx.y * g.ldy};
  KqBody<FMT>::run(g, reinterpret_cast<uint8_t *>(qlds), epi);
}

// ---- Q1_0 / PQ2_0 / PTQ1_0 on the matrix cores (the body: tern_gemv.h)



template <int FMT>
__global__ __launch_bounds__(64 * tm::waves<FMT>()) void gemv_tern_kernel(GemvArgs g) {
  extern __shared__ uint4 tlds[];
  StoreRow epi{g.y + (int64_t)blockIdx.y * g.ldy};
  tern_gemv_body<FMT>(g, tlds, epi);
}

// ---- the 512-wide Hadamard rotation (src/kernels.ts:177-227, mode 0)
//
// One 256-thread workgroup per (row, 512-block), two values per thread: the
// signs first, then the nine butterfly stages over pairs (i, i + h) in LDS
// (a + b, a - b in binary32: the same network as the reference's, so the
// same values), then binary32(1 / sqrt(512)).
__global__ __launch_bounds__(256) void hadamard_kernel(const float *x, int64_t ldx,
                                                       const float *signs, float *out, int K) {
  __shared__ float sh[512];
  const int tid = threadIdx.x;
  const int bpr = K >> 9;
  const int row = (int)blockIdx.x / bpr, c0 = ((int)blockIdx.x % bpr) * 512;
  const float *src = x + (int64_t)row * ldx + c0;
  float v0 = src[tid], v1 = src[tid + 256];
  if (signs) {
    v0 = v0 * signs[c0 + tid];
    v1 = v1 * signs[c0 + tid + 256];
  }
  sh[tid] = v0;
  sh[tid + 256] = v1;
  __syncthreads();
#pragma unroll
  for (int st = 0; st < 9; ++st) {
    const int h = 1 << st;
    const int i0 = ((tid >> st) << (st + 1)) | (tid & (h - 1));
    const float a = sh[i0], b = sh[i0 + h];
    __syncthreads();
    sh[i0] = a + b;
    sh[i0 + h] = a - b;
    __syncthreads();
  }
  const float norm = 0.04419417382415922f;
  float *dst = out + (int64_t)row * K + c0;
  dst[tid] = sh[tid] * norm;
  dst[tid + 256] = sh[tid + 256] * norm;
}

// Workgroups that are resident at once on the current GPU, cached per
// (device, kernel, dynamic LDS bytes).
int resident_blocks(const void *kernel, uint32_t lds, int threads) {
  struct Entry {
    int dev;
    const void *kernel;
    uint32_t lds;
    int blocks;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1024;
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry &e : cache)
    if (e.dev == dev && e.kernel == kernel && e.lds == lds) return e.blocks;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess ||
      per_cu < 1)
    return 1024;
  cache.push_back(Entry{dev, kernel, lds, cus * per_cu});
  return cus * per_cu;
}

namespace {

template <int FMT, int NRU>
hipError_t launch_fmt(GemvArgs g, hipStream_t stream, hipEvent_t *ev, hipEvent_t done) {
  // one pass of resident workgroups over the rows (g.blocks: the most useful)
  const int res = FMT == kW_F32
                      ? resident_blocks(reinterpret_cast<const void *>(gemv_kernel<FMT, NRU>), 0u,
                                        kGemvThreads)
                      : resident_blocks(reinterpret_cast<const void *>(gemv_lds_kernel<FMT, NRU>),
                                        (uint32_t)gemv_lds_bytes(FMT), kGemvThreads);
  g.blocks = g.blocks < res ? g.blocks : res;
  const dim3 grid((unsigned)g.blocks, (unsigned)g.M), block(kGemvThreads);
  if constexpr (FMT == kW_F32) {
    if (ev)
      hipExtLaunchKernelGGL((gemv_kernel<FMT, NRU>), grid, block, 0, stream, ev[0], ev[1], 0u, g);
    else if (done)
      hipExtLaunchKernelGGL((gemv_kernel<FMT, NRU>), grid, block, 0, stream, nullptr, done, 0u, g);
    else
      hipLaunchKernelGGL((gemv_kernel<FMT, NRU>), grid, block, 0, stream, g);
  } else {
    const uint32_t lds = (uint32_t)gemv_lds_bytes(FMT);
    if (ev)
      hipExtLaunchKernelGGL((gemv_lds_kernel<FMT, NRU>), grid, block, lds, stream, ev[0], ev[1], 0u, g);
    else if (done)
      hipExtLaunchKernelGGL((gemv_lds_kernel<FMT, NRU>), grid, block, lds, stream, nullptr, done, 0u, g);
    else
      hipLaunchKernelGGL((gemv_lds_kernel<FMT, NRU>), grid, block, lds, stream, g);
  }
  return hipGetLastError();
}

template <int FMT>
hipError_t launch_kq_mfma(GemvArgs g, hipStream_t stream, hipEvent_t *ev, hipEvent_t done) {
  using B = KqBody<FMT>;
  const size_t lds = B::lds(g.K);
  const int ntiles = (g.N + 15) / 16;
  const int res = resident_blocks(reinterpret_cast<const void *>(gemv_kq_mfma_kernel<FMT>),
                                  (uint32_t)lds, B::kThreads);
  int blocks = (ntiles + B::kWaves - 1) / B::kWaves;
  blocks = blocks < res ? blocks : res;
  // every wave of an activation row owns a hand-over slot
  blocks = blocks < g.part_cap / B::kWaves ? blocks : g.part_cap / B::kWaves;
  if (blocks < 1 || !g.part || !g.tile_cnt) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)g.M), block(B::kThreads);
  if (ev)
    hipExtLaunchKernelGGL(gemv_kq_mfma_kernel<FMT>, grid, block, lds, stream, ev[0], ev[1], 0u, g);
  else if (done)
    hipExtLaunchKernelGGL(gemv_kq_mfma_kernel<FMT>, grid, block, lds, stream, nullptr, done, 0u, g);
  else
    hipLaunchKernelGGL(gemv_kq_mfma_kernel<FMT>, grid, block, lds, stream, g);
  return hipGetLastError();
}

template <int FMT>
hipError_t launch_tern(GemvArgs g, hipStream_t stream, hipEvent_t *ev, hipEvent_t done) {
  const size_t lds = gemv_tern_lds_bytes(g.K);
  const int ntiles = (g.N + 15) / 16;
  // one workgroup per CU (its LDS holds two out), at most one per tile
  const int res = resident_blocks(reinterpret_cast<const void *>(gemv_tern_kernel<FMT>),
                                  (uint32_t)lds, 64 * tm::waves<FMT>());
  const int blocks = ntiles < res ? ntiles : res;
  const dim3 grid((unsigned)blocks, (unsigned)g.M), block(64 * tm::waves<FMT>());
  if (ev)
    hipExtLaunchKernelGGL(gemv_tern_kernel<FMT>, grid, block, lds, stream, ev[0], ev[1], 0u, g);
  else if (done)
    hipExtLaunchKernelGGL(gemv_tern_kernel<FMT>, grid, block, lds, stream, nullptr, done, 0u, g);
  else
    hipLaunchKernelGGL(gemv_tern_kernel<FMT>, grid, block, lds, stream, g);
  return hipGetLastError();
}

}  // namespace

// Per device, once (with the sampler's kernels): the matrix-core kernels'
// dynamic LDS limits.
hipError_t prepare_gemv() {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(gemv_kq_mfma_kernel<kW_Q6_K>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)KqBody<kW_Q6_K>::lds(kGemvMaxK));
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void *>(gemv_kq_mfma_kernel<kW_Q4_K>),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)KqBody<kW_Q4_K>::lds(kGemvMaxK));
  const void *tk[3] = {reinterpret_cast<const void *>(gemv_tern_kernel<kW_Q1_0>),
                       reinterpret_cast<const void *>(gemv_tern_kernel<kW_PQ2_0>),
                       reinterpret_cast<const void *>(gemv_tern_kernel<kW_PTQ1_0>)};
  for (const void *f : tk)
    if (e == hipSuccess)
      e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)gemv_tern_lds_bytes(kGemvMaxK));
  return e;
}

hipError_t launch_hadamard(const float *x, int64_t ldx, const float *signs, float *out, int M,
                           int K, hipStream_t stream) {
  const unsigned blocks = (unsigned)M * (unsigned)(K / 512);
  hipLaunchKernelGGL(hadamard_kernel, dim3(blocks), dim3(256), 0, stream, x, ldx, signs, out, K);
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs &g, hipStream_t stream, hipEvent_t *ev, hipEvent_t done) {
  const bool two = g.nru == 2;
  switch (g.type) {
    case kW_F32: return two ? launch_fmt<kW_F32, 2>(g, stream, ev, done) : launch_fmt<kW_F32, 1>(g, stream, ev, done);
    case kW_Q4_0: return two ? launch_fmt<kW_Q4_0, 2>(g, stream, ev, done) : launch_fmt<kW_Q4_0, 1>(g, stream, ev, done);
    case kW_Q4_1: return two ? launch_fmt<kW_Q4_1, 2>(g, stream, ev, done) : launch_fmt<kW_Q4_1, 1>(g, stream, ev, done);
    case kW_Q4_K: return launch_kq_mfma<kW_Q4_K>(g, stream, ev, done);
    case kW_Q6_K: return launch_kq_mfma<kW_Q6_K>(g, stream, ev, done);
    case kW_Q1_0: return launch_tern<kW_Q1_0>(g, stream, ev, done);
    case kW_PQ2_0: return launch_tern<kW_PQ2_0>(g, stream, ev, done);
    case kW_PTQ1_0: return launch_tern<kW_PTQ1_0>(g, stream, ev, done);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hs
