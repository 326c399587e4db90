// The planar Q1_0 / PQ2_0 / PTQ1_0 lm_head GEMV on the matrix cores, as a
// device-function body shared by the GEMV kernel (lmhead_kernels.hip) and the
// GEMV that samples its own rows (sampler_kernels.hip): the kernels differ
// only in what happens to each tile's results (the epilogue).
#pragma once
#include "sampler_internal.h"

#include <hip/hip_runtime.h>

namespace hs {

// ---- Q1_0 / PQ2_0 / PTQ1_0 on the matrix cores
//
// The 128-weight formats of src/gguf.ts:56-63, in the planar form the
// reference uploads (src/engine.ts:80-175): per row, nb = K / 128 blocks of
// quant bytes back to back (16 B Q1_0 sign bits, 32 B PQ2_0 2-bit codes,
// 26 B PTQ1_0 base-3 trits), and a tensor of binary16 block scales.  Weight
// = d * (c1 * code - 1) with code = the bit (Q1_0, c1 = 2), the 2-bit code
// (PQ2_0) or the trit (PTQ1_0) (src/gguf.ts:93-147, src/kernels.ts:376-700).
//
// As for Q6_K, x is held as four int8 limbs, here per 128-weight block: with
// 2^E above the block's largest |x|, x is rounded to n 2^(E - 27) and the
// limbs are n's balanced base-128 digits a_t (|a_t| <= 64), so
// x - sum_t a_t 2^(E - 6 - 7t) is at most 2^(E - 28).  A block is eight
// v_mfma_i32_16x16x64_i8 into one accumulator: B (64 x 16) holds the codes
// of 16 rows, A (16 x 64) in row 4G + t limb t of lane group G's positions,
// zero elsewhere.  The four lane groups G of a wave take four consecutive
// blocks of the same 16 rows, so the result's lane (j, G) holds the four
// exact limb sums D_t of (row j, block 4r + G), and the block's dot product
// is sum_t 2^(E - 6 - 7t) (c1 D_t - A_t), A_t the block's limb totals.
//
// The codes enter B in the order their bytes decode most cheaply; the
// position of code k = 4 w + m (byte m of B dword w) of MFMA s is tern_pos,
// and the A tables are built in that order:
//   Q1_0   dword s/2 of the block, bits 4 (s & 1) + w of each byte (a shift
//          and a mask per B dword);
//   PQ2_0  dword s of the block, codes w of each byte;
//   PTQ1_0 a 256-entry LDS table gives each byte's trits 0..3 (one dword)
//          and trit 4: MFMAs 0..5 take the four trits of four bytes, MFMAs
//          6 and 7 trit 4 of bytes 0..15 and 16..23 and the trits of the two
//          tail bytes.
namespace tm {
// waves per workgroup: the x tables are built once per workgroup; PTQ1_0
// (more registers) takes 8 so that three workgroups fit a CU
template <int FMT> constexpr int waves() { return FMT == kW_PTQ1_0 ? 8 : 16; }
constexpr int kLutBytes = 256 * 8;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc;
__device__ __forceinline__ rsrc res(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float half(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}
}  // namespace tm

__host__ __device__ inline size_t gemv_tern_lds_bytes(int K) {
  const int nb = K / 128;
  // LUT | x staged | A operands [nb][8 MFMAs][4 limbs] | zeros (the A
  // operand of the lanes outside their lane group) | limb totals | limb
  // scales | exponents | non-finite flag
  return (size_t)tm::kLutBytes + (size_t)K * 4 + (size_t)nb * 512 + 512 + (size_t)nb * 32 +
         (size_t)nb * 4 + 16;
}

// Position in the block (0..127) of code k = 4 w + m of MFMA s.
template <int FMT>
__device__ __forceinline__ int tern_pos(int s, int w, int m) {
  if constexpr (FMT == kW_Q1_0) {
    return 32 * (s >> 1) + 8 * m + 4 * (s & 1) + w;
  } else if constexpr (FMT == kW_PQ2_0) {
    return 16 * s + 4 * m + w;
  } else {
    if (s < 4) return 4 * s + w + 16 * m;        // bytes 0..15, trits 0..3
    if (s < 6) return 80 + 4 * (s - 4) + w + 8 * m;   // bytes 16..23, trits 0..3
    if (s == 6) return 64 + 4 * w + m;           // trit 4 of bytes 0..15
    if (w < 2) return 112 + 4 * w + m;           // trit 4 of bytes 16..23
    return 120 + (w - 2) + 2 * m;                // bytes 24, 25
  }
}


__device__ __forceinline__ uint32_t tern_bfi4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return (a & 0xFFu) | (b & 0xFF00u) | (c & 0xFF0000u) | (d & 0xFF000000u);
}

// A lane's share of one block (its quant dwords and the dword holding its
// binary16 scale), loaded a few items ahead of use.
template <int FMT> struct TernSlot;
template <> struct TernSlot<kW_Q1_0> { static constexpr int kDepth = 4; uint32_t q[4]; uint32_t sd; };
template <> struct TernSlot<kW_PQ2_0> { static constexpr int kDepth = 2; uint32_t q[8]; uint32_t sd; };
template <> struct TernSlot<kW_PTQ1_0> { static constexpr int kDepth = 2; uint32_t q[7]; uint32_t sd; };

// The kernel body: y row m = blockIdx.y of x W^T over the wave's tiles.  Each
// tile's 16 results go to epi.out(lane, row, value, valid) from every lane of
// the wave at once (lanes 0..15 hold them; the point is wave-uniform); the
// LDS from `tlds` on holds gemv_tern_lds_bytes(K).
template <int FMT, typename Epi>
__device__ __forceinline__ void tern_gemv_body(const GemvArgs &g, uint4 *tlds, Epi &epi) {
  using tm::v4i;
  constexpr int QB = tern_quant_bytes(FMT);
  constexpr int C1 = FMT == kW_Q1_0 ? 2 : 1;
  constexpr int D = TernSlot<FMT>::kDepth;
  constexpr int NWV = tm::waves<FMT>(), NT = 64 * NWV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = (int)blockIdx.y;
  const int K = g.K, nb = K / 128;
  uint8_t *base = reinterpret_cast<uint8_t *>(tlds);
  const uint2 *lut = reinterpret_cast<const uint2 *>(base);
  float *xs = reinterpret_cast<float *>(base + tm::kLutBytes);
  uint32_t *aop = reinterpret_cast<uint32_t *>(xs + K);   // [nb][8][4] x 4 dwords, then zeros
  v4i *atot = reinterpret_cast<v4i *>(aop + (size_t)nb * 128 + 128);
  float4 *asc = reinterpret_cast<float4 *>(atot + nb);
  int *aexp = reinterpret_cast<int *>(asc + nb);
  int *bad = aexp + nb;

  // ---- the limbs of activation row m, once per workgroup
  const float *xm = g.x + (int64_t)m * g.ldx;
  for (int i = tid; i < K; i += NT) xs[i] = xm[i];
  if constexpr (FMT == kW_PTQ1_0) {   // trits of every byte value (src/gguf.ts:111-144)
    uint2 *lw = reinterpret_cast<uint2 *>(base);
    for (int v = tid; v < 256; v += NT) {
      uint32_t t[5];
      uint32_t q = (uint32_t)v;
#pragma unroll
      for (int n = 0; n < 5; ++n) {   // trit n = ((v * 3^n mod 256) * 3) >> 8
        t[n] = (q * 3u) >> 8;
        q = (q * 3u) & 0xFFu;
      }
      lw[v] = make_uint2(t[0] | (t[1] << 8) | (t[2] << 16) | (t[3] << 24), t[4] * 0x01010101u);
    }
  }
  if (tid == 0) *bad = 0;
  if (tid < 128) aop[(size_t)nb * 128 + tid] = 0u;
  __syncthreads();
  for (int b = wave; b < nb; b += NWV) {   // block exponents
    const float v0 = xs[128 * b + lane], v1 = xs[128 * b + 64 + lane];
    float mx = fmaxf(fabsf(v0), fabsf(v1));
    const bool fin = __builtin_isfinite(v0) && __builtin_isfinite(v1);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) {
      int E = 0;
      (void)frexpf(mx, &E);   // mx < 2^E
      aexp[b] = E;
      atot[b] = v4i{0, 0, 0, 0};
      asc[b] = make_float4(ldexpf(1.f, E - 6), ldexpf(1.f, E - 13), ldexpf(1.f, E - 20),
                           ldexpf(1.f, E - 27));
    }
    if (__ballot(!fin) && lane == 0) *bad = 1;
  }
  __syncthreads();
  for (int it = tid; it < nb * 32; it += NT) {   // item (b, s, w): 4 codes
    const int b = it >> 5, s = (it >> 2) & 7, w = it & 3;
    const int E = aexp[b];
    uint32_t limb[4] = {0u, 0u, 0u, 0u};
    int At[4] = {0, 0, 0, 0};
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      // x rounded to a multiple of 2^(E - 27): |n| <= 2^27, then its
      // balanced base-128 digits, most significant first (|a_0| <= 64)
      int n = (int)rintf(ldexpf(xs[128 * b + tern_pos<FMT>(s, w, mm)], 27 - E));
      int a[4];
#pragma unroll
      for (int t = 3; t > 0; --t) {
        a[t] = ((n + 64) & 127) - 64;
        n = (n - a[t]) >> 7;
      }
      a[0] = n;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        At[t] += a[t];
        limb[t] |= ((uint32_t)a[t] & 0xFFu) << (8 * mm);
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      aop[((b * 8 + s) * 4 + t) * 4 + w] = limb[t];
      atomicAdd(reinterpret_cast<int *>(&atot[b]) + t, At[t]);
    }
  }
  __syncthreads();
  const bool nonfinite = *bad != 0;

  // ---- the wave's items: (tile of 16 rows, round r of four blocks), its
  // tiles round-robin over the grid's waves; item z + D is requested as
  // soon as item z is taken apart, so D items are in flight per wave.
  // Both resources cover their tensor rounded up to whole dwords: a dword
  // read that straddles the limit would return 0 for its valid bytes too
  // (the last PTQ1_0 block ends 2 bytes into a dword).
  const tm::rsrc rq = tm::res(g.w, (g.w_bytes + 3u) & ~3u), rs = tm::res(g.scales, (g.s_bytes + 3u) & ~3u);
  const int j = lane & 15, G = lane >> 4, tl = lane & 3;
  const bool a_live = ((lane & 15) >> 2) == G;
  const int ntiles = (g.N + 15) >> 4, nr = (nb + 3) >> 2;
  const int nw = (int)gridDim.x * NWV;
  const int first = (int)blockIdx.x * NWV + wave;
  const int Z = first < ntiles ? ((ntiles - 1 - first) / nw + 1) * nr : 0;

  auto load = [&](int z, TernSlot<FMT> &sl) {
    const int tile = first + (z / nr) * nw, b = 4 * (z % nr) + G;
    const int row = tile * 16 + j;
    const bool live = z < Z && b < nb && row < g.N;
    const uint32_t blk = (uint32_t)row * (uint32_t)nb + (uint32_t)b;
    const uint32_t so = live ? (blk * 2u) & ~3u : 0xFFFFFFF0u;   // past the resource: zeros
    sl.sd = __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0) >> (live ? 8u * (blk & 1u) * 2u : 0u);
    const uint32_t qo = blk * (uint32_t)QB;
    if constexpr (FMT == kW_Q1_0) {
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(rq, live ? qo : 0xFFFFFFF0u, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) sl.q[i] = (uint32_t)q[i];
    } else if constexpr (FMT == kW_PQ2_0) {
      const auto q0 = __builtin_amdgcn_raw_buffer_load_b128(rq, live ? qo : 0xFFFFFFF0u, 0, 0);
      const auto q1 = __builtin_amdgcn_raw_buffer_load_b128(rq, live ? qo + 16u : 0xFFFFFFF0u, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sl.q[i] = (uint32_t)q0[i];
        sl.q[4 + i] = (uint32_t)q1[i];
      }
    } else {   // 26 bytes from an even offset: seven aligned dwords
      const uint32_t a0 = qo & ~3u;
#pragma unroll
      for (int i = 0; i < 7; ++i)
        sl.q[i] = __builtin_amdgcn_raw_buffer_load_b32(rq, live ? a0 + 4u * i : 0xFFFFFFF0u, 0, 0);
    }
  };

  TernSlot<FMT> slot[D];
#pragma unroll
  for (int u = 0; u < D; ++u) load(u, slot[u]);
  float acc = 0.f;
  for (int z0 = 0; z0 < Z; z0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int z = z0 + u;
      const int tile = first + (z / nr) * nw, r = z % nr, b = 4 * r + G;
      const int row = tile * 16 + j;
      const bool bl = b < nb;
      const float d = tm::half(slot[u].sd);
      v4i D0 = v4i{0, 0, 0, 0}, D1 = v4i{0, 0, 0, 0};
      // this lane's A operand rows (limb tl of its lane group's block), or
      // the zeros: one select per item, none per MFMA
      const v4i *ab = reinterpret_cast<const v4i *>(aop) + (a_live && bl ? (size_t)b * 32 : (size_t)nb * 32) + tl;
      auto mfma = [&](int s, v4i B) {
        const v4i A = ab[s * 4];
        if (s & 1)
          D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, D1, 0, 0, 0);
        else
          D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, D0, 0, 0, 0);
      };
      if constexpr (FMT == kW_Q1_0) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const uint32_t wd = slot[u].q[s >> 1];
          v4i B;
#pragma unroll
          for (int w = 0; w < 4; ++w) B[w] = (int)((wd >> (4 * (s & 1) + w)) & 0x01010101u);
          mfma(s, B);
        }
      } else if constexpr (FMT == kW_PQ2_0) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const uint32_t wd = slot[u].q[s];
          v4i B;
#pragma unroll
          for (int w = 0; w < 4; ++w) B[w] = (int)((wd >> (2 * w)) & 0x03030303u);
          mfma(s, B);
        }
      } else {
        const uint32_t sh = ((uint32_t)(row * nb + b) * (uint32_t)QB) & 3u;
        uint32_t q[7];
#pragma unroll
        for (int i = 0; i < 6; ++i) q[i] = __builtin_amdgcn_alignbyte(slot[u].q[i + 1], slot[u].q[i], sh);
        q[6] = __builtin_amdgcn_alignbyte(0u, slot[u].q[6], sh);
        // bytes 0..15 (MFMAs 0..3 and 6), then bytes 16..25 (MFMAs 4, 5, 7)
        {
          uint2 e[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) e[i] = lut[(q[i >> 2] >> (8 * (i & 3))) & 0xFFu];
#pragma unroll
          for (int s = 0; s < 4; ++s)
            mfma(s, v4i{(int)e[4 * s].x, (int)e[4 * s + 1].x, (int)e[4 * s + 2].x,
                        (int)e[4 * s + 3].x});
          v4i B6;
#pragma unroll
          for (int w = 0; w < 4; ++w)
            B6[w] = (int)tern_bfi4(e[4 * w].y, e[4 * w + 1].y, e[4 * w + 2].y, e[4 * w + 3].y);
          mfma(6, B6);
        }
        {
          uint2 e[10];
#pragma unroll
          for (int i = 0; i < 10; ++i)
            e[i] = lut[(q[(16 + i) >> 2] >> (8 * ((16 + i) & 3))) & 0xFFu];
#pragma unroll
          for (int s = 4; s < 6; ++s) {
            const int b0 = 4 * (s - 4);
            mfma(s, v4i{(int)e[b0].x, (int)e[b0 + 1].x, (int)e[b0 + 2].x, (int)e[b0 + 3].x});
          }
          mfma(7, v4i{(int)tern_bfi4(e[0].y, e[1].y, e[2].y, e[3].y),
                      (int)tern_bfi4(e[4].y, e[5].y, e[6].y, e[7].y), (int)e[8].x, (int)e[9].x});
        }
      }
      load(z + D, slot[u]);   // the slot is free: request the item D ahead
      if (bl) {
        const v4i at = atot[b];
        const float4 sc = asc[b];
        const v4i Dt = D0 + D1;
        float val = (float)(C1 * Dt[0] - at[0]) * sc.x;
        val = fmaf((float)(C1 * Dt[1] - at[1]), sc.y, val);
        val = fmaf((float)(C1 * Dt[2] - at[2]), sc.z, val);
        val = fmaf((float)(C1 * Dt[3] - at[3]), sc.w, val);
        acc = fmaf(d, val, acc);
      }
      if (r == nr - 1) {   // the tile's last round: the four lane groups add up
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        epi.out(lane, row, nonfinite ? __builtin_nanf("") : acc, lane < 16 && row < g.N && z < Z);
        acc = 0.f;
      }
    }
  }
}

}  // namespace hs
