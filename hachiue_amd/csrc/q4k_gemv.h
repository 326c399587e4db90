// The Q4_K lm_head GEMV on the matrix cores, as a device-function body (the
// kernel in lmhead_kernels.hip adds the epilogue that stores each tile's
// results), in the form of the Q6_K body (q6k_gemv.h): tiles of 16 rows per
// wave, slabs of super-blocks read straight into an LDS ring, integer limbs
// of x and v_mfma_i32_16x16x64_i8.
#pragma once
#include "sampler_internal.h"

#include <hip/hip_runtime.h>

namespace hs {

// ---- Q4_K on the matrix cores
//
// A Q4_K super-block (144 bytes, 256 weights; src/gguf.ts:174-204) holds d
// and dmin (binary16), twelve bytes of 6-bit scales sc_j and minima m_j of
// its eight 32-weight sub-blocks, and 128 bytes of 4-bit q: byte 32 p + l
// holds weight 64 p + l in its low nibble (sub-block 2 p) and weight 64 p +
// 32 + l in its high nibble (sub-block 2 p + 1).  A weight is
// d sc_j q - dmin m_j.
//
// x is held as four int8 limbs per group of 16 positions, as for Q6_K (2^E
// above the group's largest |x|, a_t = rint(r_{t-1} 2^(6 + 7t - E)), |a_t| <=
// 64, remainder below 2^(E - 28)).  MFMA i of a row covers positions 64 i ..
// 64 i + 63, its super-block's pair p = i % 4: lane (j, G) holds in B the 16
// q of positions 64 i + 16 G .. + 15 of row j (bytes 32 p + 16 (G & 1) ..
// + 15 of the quants, low nibbles for G < 2, high for G >= 2), so its
// sub-block is 2 p + (G >> 1); A holds in row 4 G + t limb t of group 4 i +
// G.  The lane receives the four integer limb sums D_t of its (row, group),
// and adds d sc 2^(E - 6) sum_t 2^(-7t) D_t - dmin m (sum of the group's x);
// a group's 2^(E - 6) and sum of x are one 8-byte LDS record.
//
// Work and reads as in the Q6_K body, with a slab of one super-block (16
// rows x 144 bytes: rows are 16-byte aligned) and a ring of three: two slabs
// in flight per wave while one is taken apart, the ring of 8 waves and the x
// tables within half the CU's LDS at K 4096.  Rows 144 bytes (36 banks)
// apart: the 16 rows' 16-byte reads of a lane group meet no bank twice.
namespace q4m {
constexpr int kSB = 1;                               // super-blocks per slab
constexpr int kNB = 3;                               // ring depth (slabs per wave)
constexpr int kRowChunks = 9;                        // 16-byte chunks per row
constexpr int kSlabRowBytes = 16 * kRowChunks;       // 144
constexpr int kLoads = (16 * kRowChunks + 63) / 64;  // 1 KiB loads per slab: 3, the last
constexpr int kLastLanes = 16 * kRowChunks - 64 * (kLoads - 1);   //   by 16 lanes
constexpr int kSlabBytes = 16 * kSlabRowBytes;       // 2304
constexpr int kWaves = 8;                            // per workgroup, 2 workgroups per CU
constexpr int kThreads = 64 * kWaves;
typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}
// sub-block j's 6-bit scale and minimum from the super-block's bytes 4..15
// (w1, w2, w3: its dwords 1, 2, 3; src/gguf.ts:178-186)
__device__ __forceinline__ void scale_min(uint32_t w1, uint32_t w2, uint32_t w3, int j, uint32_t &sc,
                                          uint32_t &mn) {
  if (j < 4) {
    sc = (w1 >> (8 * j)) & 63u;
    mn = (w2 >> (8 * j)) & 63u;
  } else {
    const int s = 8 * (j - 4);
    const uint32_t b = (w3 >> s) & 0xFFu;
    sc = (b & 0x0Fu) | (((w1 >> s) >> 6 & 3u) << 4);
    mn = (b >> 4) | (((w2 >> s) >> 6 & 3u) << 4);
  }
}
}  // namespace q4m

__host__ __device__ inline size_t gemv_q4k_mfma_lds_bytes(int K) {
  // A operands: 256 B per 64 positions; per group of 16 positions 2^(E - 6)
  // and its sum of x (float2); the slab rings
  return (size_t)(K / 64) * 256 + (size_t)(K / 16) * 8 +
         (size_t)q4m::kWaves * q4m::kNB * q4m::kSlabBytes;
}

// The body of a kernel of 2 workgroups per CU (16 waves: at most 128 VGPRs)
// and q4m::kThreads threads: activation row blockIdx.y, its LDS at `lds`
// (gemv_q4k_mfma_lds_bytes(K)).  Each row's result goes to
// epi.out(lane, row, value, valid), called by every lane of a wave at once,
// lanes 0..15 holding the 16 rows of a tile (valid: lane < 16, row < N).
// The tensor is 16-byte aligned (then so is every row).
template <class Epi>
__device__ __forceinline__ void q4k_gemv_body(const GemvArgs &g, uint8_t *lds, Epi &epi) {
  constexpr int NB = q4m::kNB;
  using namespace q4m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = (int)blockIdx.y;
  const int K = g.K, NG = K / 16, NS = K / 256;
  v4i *aop = reinterpret_cast<v4i *>(lds);                        // [K/64][4 G][4 t]
  float2 *pgx = reinterpret_cast<float2 *>(lds + (size_t)(K / 64) * 256);   // [K/16]
  uint8_t *ring = reinterpret_cast<uint8_t *>(pgx + NG) + (size_t)wave * NB * kSlabBytes;

  // Work, as in the Q6_K body: whole tiles round-robin over the waves for as
  // many full rounds as there are; the tiles left are cut into P slab ranges
  // each, whose partial sums the last part to count in adds in part order.
  const int nw = (int)gridDim.x * q4m::kWaves;
  const int wg = (int)blockIdx.x * q4m::kWaves + wave;
  const int ntiles = (g.N + 15) >> 4;
  const int nsl = (NS + kSB - 1) / kSB;
  const int rfull = ntiles / nw, tail = ntiles - rfull * nw;
  int P = tail > 0 ? nw / tail : 1;
  P = P < nsl ? P : nsl;
  const bool has_part = tail > 0 && wg < tail * P;
  const int ptt = wg / P, pidx = wg - ptt * P;
  const int p0 = pidx * nsl / P, p1 = (pidx + 1) * nsl / P;
  const int items = rfull * nsl + (has_part ? p1 - p0 : 0);
  auto item = [&](int z, int &tile, int &sl) {
    if (z < rfull * nsl) {
      tile = wg + (z / nsl) * nw;
      sl = z % nsl;
      return sl == nsl - 1;
    }
    tile = rfull * nw + ptt;
    sl = p0 + (z - rfull * nsl);
    return sl == p1 - 1;
  };
  const uint32_t RB = g.row_bytes;
  const int j = lane & 15, G = lane >> 4;
  const bool a_live = ((lane & 15) >> 2) == G;

  // reads into LDS from inline assembly, as in the Q6_K body (the compiler
  // cannot tell the ring's buffers apart); the waits below are explicit
  const uint64_t wbase = reinterpret_cast<uint64_t>(g.w);
  const v4i rs = v4i{(int)(uint32_t)wbase, (int)(uint32_t)(wbase >> 32),
                     (int)((g.w_bytes + 15u) & ~15u), 0x00020000};
  auto issue = [&](int z, uint8_t *dst) {   // slab z of this wave into dst
    int tile, sl;
    (void)item(z, tile, sl);
#pragma unroll
    for (int c = 0; c < kLoads; ++c) {
      const int q = c * 64 + lane, rj = q / kRowChunks, cc = q % kRowChunks;
      const int row = tile * 16 + rj;
      const uint32_t off =
          row < g.N ? (uint32_t)row * RB + 144u * (uint32_t)sl + 16u * (uint32_t)cc : 0xFFFFFFF0u;
      const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) uint8_t *)(dst + c * 1024)));
      if (c + 1 < kLoads || lane < kLastLanes) {
        uint32_t keep;
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\t"
            "buffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
            : "=&s"(keep)
            : "s"(m0), "v"(off), "s"(rs)
            : "memory");
      }
    }
  };

  float acc = 0.f;
  // slab z sits in ring buffer z % NB, its loads issued NB - 1 slabs earlier;
  // the first ones go out before the x tables are built
  for (int z = 0; z < items && z < NB - 1; ++z) issue(z, ring + z * kSlabBytes);
  // limbs of this activation row, once per workgroup; a non-finite element
  // makes the row's results NaN
  __shared__ int nonfin;
  if (tid == 0) nonfin = 0;
  __syncthreads();
  const float *xm = g.x + (int64_t)m * g.ldx;
  for (int gi = tid; gi < NG; gi += q4m::kThreads) {
    float xv[16], mx = 0.f, sx = 0.f;
    bool fin = true;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      xv[b] = xm[16 * gi + b];
      mx = fmaxf(mx, fabsf(xv[b]));
      sx += xv[b];
      fin = fin && __builtin_isfinite(xv[b]);
    }
    if (!fin) nonfin = 1;
    int E = 0;
    (void)frexpf(mx, &E);   // mx < 2^E
    uint32_t limb[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int w = 0; w < 4; ++w) limb[t][w] = 0u;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      float r = xv[b];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float a = rintf(ldexpf(r, 6 + 7 * t - E));
        r -= ldexpf(a, E - 6 - 7 * t);   // exact: a 2^(E-6-7t) is within half a step of r
        limb[t][b >> 2] |= ((uint32_t)(int)a & 0xFFu) << (8 * (b & 3));
      }
    }
    const int mi = gi >> 2, Gg = gi & 3;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      aop[(mi * 4 + Gg) * 4 + t] = v4i{(int)limb[t][0], (int)limb[t][1], (int)limb[t][2], (int)limb[t][3]};
    pgx[gi] = make_float2(ldexpf(1.f, E - 6), sx);
  }
  __syncthreads();
  const bool nan_out = nonfin != 0;
  const int hi = G >> 1;                  // high nibbles
  const uint32_t qoff = 16u + 16u * (uint32_t)(G & 1);   // within a pair's 32 quant bytes
  for (int z = 0; z < items; ++z) {
    const uint8_t *cur = ring + (z % NB) * kSlabBytes;
    if (z + NB - 1 < items) {
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the buffer's reads are done
      issue(z + NB - 1, ring + ((z + NB - 1) % NB) * kSlabBytes);
    }
    // slab z has arrived once at most the later slabs' loads are in flight
    // (kLoads each; vector-memory loads complete in order, a y store among
    // them only makes the wait longer)
    static_assert(NB == 3 && 2 * kLoads < 16, "two later slabs, vmcnt below 16");
    if (z + 2 < items)
      __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * kLoads));   // vmcnt(2 kLoads)
    else if (z + 1 < items)
      __builtin_amdgcn_s_waitcnt(0x0F70 | kLoads);         // vmcnt(kLoads)
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
    asm volatile("" ::: "memory");
    int tile, sl;
    const bool seg_end = item(z, tile, sl);
    const int row = tile * 16 + j;
    const uint8_t *rowb = cur + j * kSlabRowBytes;
    {
      const int sbk = sl;
      const uint4 hd = *reinterpret_cast<const uint4 *>(rowb);   // d, dmin, the scales
      const float d = q4m::h2f(hd.x), dmin = q4m::h2f(hd.x >> 16);
      float accd = 0.f, accm = 0.f;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint4 qb = *reinterpret_cast<const uint4 *>(rowb + qoff + 32 * p);
        const uint32_t sh = 4u * (uint32_t)hi;
        const v4i bq = v4i{(int)((qb.x >> sh) & 0x0F0F0F0Fu), (int)((qb.y >> sh) & 0x0F0F0F0Fu),
                           (int)((qb.z >> sh) & 0x0F0F0F0Fu), (int)((qb.w >> sh) & 0x0F0F0F0Fu)};
        const int mi = 4 * sbk + p;
        const v4i al = aop[(mi * 4 + G) * 4 + (lane & 3)];
        const v4i a = a_live ? al : v4i{0, 0, 0, 0};
        const v4i dq = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bq, v4i{0, 0, 0, 0}, 0, 0, 0);
        const int gi = 4 * mi + G;
        const float2 gx = pgx[gi];
        float val = fmaf((float)dq[1], 0x1p-7f, (float)dq[0]);
        val = fmaf((float)dq[2], 0x1p-14f, val);
        val = fmaf((float)dq[3], 0x1p-21f, val);
        uint32_t sc, mn;
        q4m::scale_min(hd.y, hd.z, hd.w, 2 * p + hi, sc, mn);
        accd = fmaf((float)sc, val * gx.x, accd);   // times a power of two: exact
        accm = fmaf((float)mn, gx.y, accm);
      }
      acc = fmaf(d, accd, acc);
      acc = fmaf(-dmin, accm, acc);
    }
    if (seg_end) {   // the four lane groups of a row add up
      acc += __shfl_xor(acc, 16);
      acc += __shfl_xor(acc, 32);
      if (z < rfull * nsl || P == 1) {
        epi.out(lane, row, nan_out ? __builtin_nanf("") : acc, lane < 16 && row < g.N);
      } else {
        float *pm = g.part + ((int64_t)m * g.part_cap + wg) * 16;   // slot ptt * P + pidx == wg
        if (lane < 16)
          __hip_atomic_store(pm + lane, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the sums are out
        uint32_t *cnt = g.tile_cnt + (int64_t)m * g.part_cap + ptt;
        uint32_t old = 0;
        if (lane == 0)
          old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old == (uint32_t)(P - 1)) {   // the last part: add all P in order
          const float *p0p = g.part + ((int64_t)m * g.part_cap + (int64_t)ptt * P) * 16;
          float sum = 0.f;
          for (int q = 0; q < P; ++q)
            sum += lane < 16 ? __hip_atomic_load(p0p + q * 16 + lane, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)
                             : 0.f;
          epi.out(lane, row, nan_out ? __builtin_nanf("") : sum, lane < 16 && row < g.N);
          if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      acc = 0.f;
    }
  }
}

}  // namespace hs
