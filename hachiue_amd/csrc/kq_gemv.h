// The K-quant lm_head GEMVs on the matrix cores (Q4_K: q4k_gemv.h, Q6_K:
// q6k_gemv.h) behind one name, for the kernels built on either body: the
// plain GEMV (lmhead_kernels.hip) and the GEMVs that keep their rows' argmax
// or sample them (sampler_kernels.hip).
#pragma once
#include "q4k_gemv.h"
#include "q6k_gemv.h"

namespace hs {

// kWaves and kThreads per workgroup (2 workgroups per CU), the body's LDS
// (lds(K)), where its slab rings start (ring_off(K); after the body's loop
// they are free) and their bytes (kRingBytes), and the body itself (run).
template <int FMT>
struct KqBody;

template <>
struct KqBody<kW_Q6_K> {
  static constexpr int kWaves = q6m::kWaves, kThreads = q6m::kThreads;
  static constexpr size_t kRingBytes = (size_t)q6m::kWaves * q6m::kNB * q6m::kSlabBytes;
  __host__ __device__ static size_t lds(int K) { return gemv_q6k_mfma_lds_bytes(K); }
  __host__ __device__ static size_t ring_off(int K) {   // the A tables, then the rings
    return (size_t)(K / 64) * 256 + (size_t)(K / 16) * 32;
  }
  template <class Epi>
  __device__ __forceinline__ static void run(const GemvArgs &g, uint8_t *l, Epi &epi) {
    q6k_gemv_body(g, l, epi);
  }
};

template <>
struct KqBody<kW_Q4_K> {
  static constexpr int kWaves = q4m::kWaves, kThreads = q4m::kThreads;
  static constexpr size_t kRingBytes = (size_t)q4m::kWaves * q4m::kNB * q4m::kSlabBytes;
  __host__ __device__ static size_t lds(int K) { return gemv_q4k_mfma_lds_bytes(K); }
  __host__ __device__ static size_t ring_off(int K) {   // the A tables and sums, then the rings
    return (size_t)(K / 64) * 256 + (size_t)(K / 16) * 8;
  }
  template <class Epi>
  __device__ __forceinline__ static void run(const GemvArgs &g, uint8_t *l, Epi &epi) {
    q4k_gemv_body(g, l, epi);
  }
};

static_assert(KqBody<kW_Q6_K>::kWaves * 2 == kGemvWavesPerCU &&
                  KqBody<kW_Q4_K>::kWaves * 2 == kGemvWavesPerCU,
              "the hand-over slots: 2 workgroups per CU");

}  // namespace hs
