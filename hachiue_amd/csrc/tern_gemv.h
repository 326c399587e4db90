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
// of 16 rows, A (16 x 64) in row 4G + t limb t (times c1) of lane group G's
// positions, zero elsewhere, and the accumulator starts at -A_t, A_t the
// block's limb totals.  The four lane groups G of a wave take four
// consecutive blocks of the same 16 rows, so the result's lane (j, G) holds
// the four exact sums D_t = c1 sum a_t code - A_t of (row j, block 4r + G),
// and the block's dot product is sum_t 2^(E - 6 - 7t) D_t, taken as two
// exact integer pairs (128 D_0 + D_1, 128 D_2 + D_3).  Q1_0 (c1 = 2) takes
// E one higher so that the doubled limbs stay within int8.
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
// waves per workgroup: one workgroup per CU (the LDS below holds two out),
// which builds the x tables once for its 16 waves
template <int FMT> constexpr int waves() { return 16; }
constexpr int kLutBytes = 256 * 8;
// the items' partial results of one chunk of a workgroup's tiles, and the
// chunk's binary16 block scales (at most 16 rows x 4 nr blocks x 2 bytes a
// tile, half the partials' 16 x 64 x 4 bytes a round)
constexpr int kPartBytes = 64 * 1024;
constexpr int kScaleBytes = kPartBytes / 2;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc;
__device__ __forceinline__ rsrc res(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float half(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}
}  // namespace tm

// blocks of a row rounded up to whole rounds of four
__host__ __device__ inline int tern_nbp(int K) { return 4 * ((K / 128 + 3) / 4); }

__host__ __device__ inline size_t gemv_tern_lds_bytes(int K) {
  const int nbp = tern_nbp(K);
  // LUT | A operands [nbp][8 MFMAs][4 limbs] | zeros (the A operand of the
  // lanes outside their lane group) | limb totals | the two limb-pair
  // scales | non-finite flags (one a wave) | partial results | block scales
  return (size_t)tm::kLutBytes + (size_t)nbp * 512 + 512 + (size_t)nbp * 16 + (size_t)nbp * 8 +
         16 * 4 + tm::kPartBytes + tm::kScaleBytes + 16;   // (+ the pad lanes' reads past the last row)
}

// Tiles of 16 rows that one chunk of a workgroup may hold (its items'
// partial results fill at most kPartBytes).
__host__ __device__ inline int tern_chunk_tiles(int K) {
  const int nr = tern_nbp(K) / 4;
  return tm::kPartBytes / (nr * 64 * 4);
}

// The most tiles one wave hands to the epilogue, on a grid of `blocks`
// workgroups of nw waves.
__host__ __device__ inline int tern_out_tiles_max(int N, int K, int blocks, int nw) {
  const int ntiles = (N + 15) / 16;
  const int wg = (ntiles + blocks - 1) / blocks;
  const int cm = tern_chunk_tiles(K);
  const int nch = (wg + cm - 1) / cm;
  if (nch == 0) return 0;
  const int ct = (wg + nch - 1) / nch;
  return nch * ((ct + nw - 1) / nw);
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


// The inverse of tern_pos: MFMA s, B dword w and byte m of position p.
template <int FMT>
__device__ __forceinline__ void tern_inv(int p, int &s, int &w, int &m) {
  if constexpr (FMT == kW_Q1_0) {
    s = 2 * (p >> 5) + ((p >> 2) & 1);
    m = (p >> 3) & 3;
    w = p & 3;
  } else if constexpr (FMT == kW_PQ2_0) {
    s = p >> 4;
    m = (p >> 2) & 3;
    w = p & 3;
  } else {
    if (p < 64) {
      s = (p >> 2) & 3; w = p & 3; m = p >> 4;
    } else if (p < 80) {
      s = 6; w = (p - 64) >> 2; m = (p - 64) & 3;
    } else if (p < 112) {
      s = 4 + (((p - 80) >> 2) & 1); w = (p - 80) & 3; m = (p - 80) >> 3;
    } else if (p < 120) {
      s = 7; w = (p - 112) >> 2; m = (p - 112) & 3;
    } else {
      s = 7; w = 2 + ((p - 120) & 1); m = (p - 120) >> 1;
    }
  }
}

__device__ __forceinline__ uint32_t tern_bfi4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return (a & 0xFFu) | (b & 0xFF00u) | (c & 0xFF0000u) | (d & 0xFF000000u);
}

// A lane's share of one block (its quant dwords), loaded a few items ahead
// of use.
template <int FMT> struct TernSlot;
// (depths measured at 151936 x 2048, interleaved runs, kernel median: Q1_0
// 6 -> 4 took 17.6 -> 15.9 us, PTQ1_0 3 -> 2 25.4 -> 23.4 us; PQ2_0 from 2
// to 4 within 0.4 us; deeper was slower for all three)
template <> struct TernSlot<kW_Q1_0> { static constexpr int kDepth = 4; uint32_t q[4]; };
template <> struct TernSlot<kW_PQ2_0> { static constexpr int kDepth = 4; uint32_t q[8]; };
template <> struct TernSlot<kW_PTQ1_0> { static constexpr int kDepth = 2; uint32_t q[7]; };

// The kernel body: y row m = blockIdx.y of x W^T.  Workgroup b of the grid
// takes the tiles b, b + G, b + 2G, ... of the T tiles of 16 rows, in
// chunks of at most tern_chunk_tiles; an item is (tile, round r of four
// blocks), and the chunk's items go round-major (every tile's round 0, then
// round 1, ...) to its waves in equal contiguous runs, so that a wave keeps
// one round's A operands in registers over many tiles.  Each item's 64
// per-lane partial sums go to LDS; after a barrier each tile's 16 results
// (the sum over rounds, then over the four lane groups, in that fixed
// order) go to epi.out(lane, row, value, valid) from every lane of one wave
// at once (lanes 0..15 hold them; the point is wave-uniform).  The LDS from
// `tlds` on holds gemv_tern_lds_bytes(K).
template <int FMT, typename Epi>
__device__ __forceinline__ void tern_gemv_body(const GemvArgs &g, uint4 *tlds, Epi &epi) {
  using tm::v4i;
  constexpr int QB = tern_quant_bytes(FMT);
  constexpr int C1 = FMT == kW_Q1_0 ? 2 : 1;
  constexpr int D = TernSlot<FMT>::kDepth;
  constexpr int NWV = tm::waves<FMT>(), NT = 64 * NWV;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: the item cursors stay scalar)
  const int m = (int)blockIdx.y;
  const int K = g.K, nb = K / 128, nbp = tern_nbp(K), nr = nbp / 4;
  static_assert(kGemvMaxK % NT == 0, "x in whole passes");
  uint8_t *base = reinterpret_cast<uint8_t *>(tlds);
  const uint2 *lut = reinterpret_cast<const uint2 *>(base);
  uint32_t *aop = reinterpret_cast<uint32_t *>(base + tm::kLutBytes);   // [nbp][8][4] x 4 dwords, then zeros
  v4i *atot = reinterpret_cast<v4i *>(aop + (size_t)nbp * 128 + 128);
  float2 *asc = reinterpret_cast<float2 *>(atot + nbp);
  int *badw = reinterpret_cast<int *>(asc + nbp);   // per wave: a non-finite x seen
  float *part = reinterpret_cast<float *>(badw + NWV);
  uint8_t *sclb = reinterpret_cast<uint8_t *>(part) + tm::kPartBytes;   // [ct][16 rows][nb] binary16
  const uint16_t *scl = reinterpret_cast<const uint16_t *>(sclb);

  // ---- this workgroup's tiles and their chunks
  const int ntiles = (g.N + 15) >> 4;
  // (tiles b, b + G, b + 2G, ...: at any time the grid's loads fall in a
  // few contiguous stretches of the weights, which the DRAM pages serve
  // better than one stretch per workgroup)
  const int G = (int)gridDim.x, bx = (int)blockIdx.x;
  const int nt_wg = bx < ntiles ? (ntiles - 1 - bx) / G + 1 : 0, cmax = tern_chunk_tiles(K);
  const int nch = (nt_wg + cmax - 1) / cmax;

  // ---- lane constants.  Lane (j, G) takes row j of the tile and block
  // 4 r + G of round r; its quant dword offset is a per-lane part plus a
  // wave-uniform part per item.  Both resources cover their tensor rounded
  // up to whole dwords: a dword read that straddles the limit would return 0
  // for its valid bytes too (the last PTQ1_0 block ends 2 bytes into a
  // dword).  Rows past N read past the resource: zeros.
  const tm::rsrc rq = tm::res(g.w, (g.w_bytes + 3u) & ~3u), rs = tm::res(g.scales, (g.s_bytes + 3u) & ~3u);
  const int j = lane & 15, lg = lane >> 4, tl = lane & 3;
  const bool a_live = ((lane & 15) >> 2) == lg;
  const uint32_t jb = (uint32_t)(j * nb + lg);
  const uint32_t shq = (jb * (uint32_t)QB) & 3u;   // PTQ1_0: 2 on odd blocks
  const uint32_t lb_q = jb * (uint32_t)QB - shq;

  // item (t, r) of the chunk starting at tile c0: its loads (zeros when
  // not `live`, so that every path issues the same loads and the waits
  // count them exactly)
  auto load = [&](int c0, int t, int r, TernSlot<FMT> &sl, bool live) {
    const uint32_t ub = (uint32_t)(bx + (c0 + t) * G) * 16u * (uint32_t)nb + 4u * (uint32_t)r;
    uint32_t vq = lb_q + ub * (uint32_t)QB;
    if (!live || (4 * r + 4 > nb && lg >= nb - 4 * r)) vq = 0xFFFFFF00u;   // past the row's last block: zeros
    if constexpr (FMT == kW_Q1_0) {
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(rq, vq, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) sl.q[i] = (uint32_t)q[i];
    } else if constexpr (FMT == kW_PQ2_0) {
      const auto q0 = __builtin_amdgcn_raw_buffer_load_b128(rq, vq, 0, 0);
      const auto q1 = __builtin_amdgcn_raw_buffer_load_b128(rq, vq + 16u, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sl.q[i] = (uint32_t)q0[i];
        sl.q[4 + i] = (uint32_t)q1[i];
      }
    } else {   // 26 bytes from an even offset: seven aligned dwords
      const auto q0 = __builtin_amdgcn_raw_buffer_load_b128(rq, vq, 0, 0);
      const auto q1 = __builtin_amdgcn_raw_buffer_load_b96(rq, vq + 16u, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) sl.q[i] = (uint32_t)q0[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) sl.q[4 + i] = (uint32_t)q1[i];
    }
  };
  // the chunk's block scales: its tiles' 16 rows are contiguous in the
  // scale tensor, 32 nb bytes a tile; piece p (16 bytes) of the chunk is
  // byte 16 p of the LDS copy (two pieces a thread at most)
  constexpr int SP = tm::kScaleBytes / 16 / NT;
  auto scale_load = [&](int c0, int ct, uint4 (&sv)[SP]) {
#pragma unroll
    for (int k = 0; k < SP; ++k) {
      const int p = tid + k * NT, tt = p / (2 * nb), q = p - tt * 2 * nb;
      const uint32_t off = tt < ct ? (uint32_t)(bx + (c0 + tt) * G) * 32u * (uint32_t)nb + 16u * (uint32_t)q
                                   : 0xFFFFFF00u;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
      sv[k] = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
    }
  };
  auto scale_store = [&](int ct, const uint4 (&sv)[SP]) {
#pragma unroll
    for (int k = 0; k < SP; ++k)
      if (tid + k * NT < ct * 2 * nb) reinterpret_cast<uint4 *>(sclb)[tid + k * NT] = sv[k];
  };
  // the wave's items of chunk c: [i0, i1) of the chunk's CT * nr
  auto chunk = [&](int c, int &c0, int &ct, int &i0, int &n) {
    c0 = (int)((int64_t)c * nt_wg / nch);
    ct = (int)((int64_t)(c + 1) * nt_wg / nch) - c0;
    const int items = ct * nr;
    i0 = (int)((int64_t)wave * items / NWV);
    n = (int)((int64_t)(wave + 1) * items / NWV) - i0;
  };

  // ---- x (wave w takes blocks w and w + 16, two values a lane), then the
  // first chunk's first kPre loads, both before the tables are built (the
  // loads complete in order: x is waited for alone); the chunk's other
  // first loads follow the tables
  constexpr int XB = kGemvMaxK / 128 / NWV;
  static_assert(XB * 128 * NWV == kGemvMaxK, "x in whole blocks per wave");
  constexpr int kPre = D < 2 ? D : 2;
  const float *xm = g.x + (int64_t)m * g.ldx;
  float xv[XB][2];
#pragma unroll
  for (int k = 0; k < XB; ++k) {
    const int b = wave + k * NWV;
    xv[k][0] = b < nb ? xm[128 * b + lane] : 0.f;
    xv[k][1] = b < nb ? xm[128 * b + 64 + lane] : 0.f;
  }
  TernSlot<FMT> slot[D];
  int c0 = 0, ct = 1, i0 = 0, n = 0;
  if (nch > 0) chunk(0, c0, ct, i0, n);
  uint4 sv[SP];
  scale_load(c0, nch > 0 ? ct : 0, sv);
  int lt0 = i0 % ct, lr0 = i0 / ct;
#pragma unroll
  for (int u = 0; u < kPre; ++u) {
    load(c0, lt0, lr0, slot[u], u < n);
    if (++lt0 == ct) { lt0 = 0; ++lr0; }
  }

  // ---- the tables of activation row m, once per workgroup: each block's
  // limbs, permuted into the A operands' byte order, their totals and the
  // limb-pair scales (pad blocks past nb: zeros)
  if constexpr (FMT == kW_PTQ1_0) {   // trits of every byte value (src/gguf.ts:111-144)
    uint2 *lw = reinterpret_cast<uint2 *>(base);
    for (int v = tid; v < 256; v += NT) {
      uint32_t t[5];
      uint32_t q = (uint32_t)v;
#pragma unroll
      for (int k = 0; k < 5; ++k) {   // trit k = ((v * 3^k mod 256) * 3) >> 8
        t[k] = (q * 3u) >> 8;
        q = (q * 3u) & 0xFFu;
      }
      lw[v] = make_uint2(t[0] | (t[1] << 8) | (t[2] << 16) | (t[3] << 24), t[4] * 0x01010101u);
    }
  }
  if (tid < 128) aop[(size_t)nbp * 128 + tid] = 0u;
  uint8_t *aob = reinterpret_cast<uint8_t *>(aop);
  bool fin = true;
#pragma unroll
  for (int k = 0; k < XB; ++k) {
    const int b = wave + k * NWV;
    if (b >= nbp) break;
    if (b >= nb) {   // pad block
      aop[(size_t)b * 128 + lane] = 0u;
      aop[(size_t)b * 128 + 64 + lane] = 0u;
      if (lane == 0) {
        atot[b] = v4i{0, 0, 0, 0};
        asc[b] = make_float2(0.f, 0.f);
      }
      continue;
    }
    const float v0 = xv[k][0], v1 = xv[k][1];
    fin = fin && __builtin_isfinite(v0) && __builtin_isfinite(v1);
    float mx = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    int E = 0;
    (void)frexpf(mx, &E);   // mx < 2^E
    // Q1_0 takes its limbs doubled (c1 = 2 folded into A): one more bit of
    // headroom keeps 2 a within int8
    E += C1 == 2 ? 1 : 0;
    uint32_t lo = 0u, hi = 0u;   // limb totals, two to a word, each + 64 per value
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // x rounded to a multiple of 2^(E - 27): |n| <= 2^27, then its
      // balanced base-128 digits, most significant first (|a_0| <= 64)
      const int p = 64 * h + lane;
      int nn = (int)rintf(ldexpf(h ? v1 : v0, 27 - E));
      int a[4];
#pragma unroll
      for (int t = 3; t > 0; --t) {
        a[t] = ((nn + 64) & 127) - 64;
        nn = (nn - a[t]) >> 7;
      }
      a[0] = nn;
      int s_, w_, m_;
      tern_inv<FMT>(p, s_, w_, m_);
      uint8_t *dst = aob + (size_t)b * 512 + s_ * 64 + 4 * w_ + m_;
#pragma unroll
      for (int t = 0; t < 4; ++t) dst[16 * t] = (uint8_t)(C1 * a[t]);
      lo += (uint32_t)(a[0] + 64) | ((uint32_t)(a[1] + 64) << 16);
      hi += (uint32_t)(a[2] + 64) | ((uint32_t)(a[3] + 64) << 16);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      lo += __shfl_xor(lo, o);
      hi += __shfl_xor(hi, o);
    }
    if (lane == 0) {
      atot[b] = v4i{(int)(lo & 0xFFFFu) - 128 * 64, (int)(lo >> 16) - 128 * 64,
                    (int)(hi & 0xFFFFu) - 128 * 64, (int)(hi >> 16) - 128 * 64};
      asc[b] = make_float2(ldexpf(1.f, E - 13), ldexpf(1.f, E - 27));
    }
  }
  fin = __all(fin);
  if (lane == 0) badw[wave] = fin ? 0 : 1;
  scale_store(nch > 0 ? ct : 0, sv);
#pragma unroll
  for (int u = kPre; u < D; ++u) {
    load(c0, lt0, lr0, slot[u], u < n);
    if (++lt0 == ct) { lt0 = 0; ++lr0; }
  }
  __syncthreads();
  bool nonfinite = false;
#pragma unroll
  for (int w = 0; w < NWV; ++w) nonfinite = nonfinite || badw[w] != 0;

  // ---- the chunks
  for (int c = 0; c < nch; ++c) {
    if (c > 0) {   // the previous chunk's results are out: its partials and scales are free
      __syncthreads();
      chunk(c, c0, ct, i0, n);
      scale_load(c0, ct, sv);
      scale_store(ct, sv);
      __syncthreads();
      int lt = i0 % ct, lr = i0 / ct;
#pragma unroll
      for (int u = 0; u < D; ++u) {
        load(c0, lt, lr, slot[u], u < n);
        if (++lt == ct) { lt = 0; ++lr; }
      }
    }
    // load cursor (D items ahead) and item cursor
    int lt = (i0 + D) % ct, lr = (i0 + D) / ct;
    int t = i0 % ct, r = i0 / ct;
    int cur_r = -1;
    v4i A[8], Cn = v4i{0, 0, 0, 0};
    float sH = 0.f, sL = 0.f;
    for (int z0 = 0; z0 < n; z0 += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const int z = z0 + u;
        // (every pass issues its D loads, in range or not: the waits then
        // count exactly the later items' loads)
        if (z < n) {
        if (r != cur_r) {   // round r's A operands, limb totals and scales
          cur_r = r;
          const int b = 4 * r + lg;
          const v4i *ab = reinterpret_cast<const v4i *>(aop) + (a_live ? (size_t)b * 32 : (size_t)nbp * 32) + tl;
#pragma unroll
          for (int s = 0; s < 8; ++s) A[s] = ab[s * 4];
          const v4i at = atot[b];
          Cn = v4i{-at[0], -at[1], -at[2], -at[3]};
          const float2 sc = asc[b];
          sH = sc.x;
          sL = sc.y;
        }
        // lane (j, G) of the result: c1 D_t - A_t of (row j, block 4 r + G)
        v4i acc = Cn;
        auto mfma = [&](int s, v4i B) { acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[s], B, acc, 0, 0, 0); };
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
          uint32_t q[7];
#pragma unroll
          for (int i = 0; i < 6; ++i) q[i] = __builtin_amdgcn_alignbyte(slot[u].q[i + 1], slot[u].q[i], shq);
          q[6] = __builtin_amdgcn_alignbyte(0u, slot[u].q[6], shq);
          // bytes 0..15 four at a time (MFMAs 0..3, their trits 4 to MFMA 6),
          // then bytes 16..25 (MFMAs 4, 5, 7)
          auto byte = [&](int i) { return lut[(q[i >> 2] >> (8 * (i & 3))) & 0xFFu]; };
          v4i B6;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const uint2 e0 = byte(4 * s), e1 = byte(4 * s + 1), e2 = byte(4 * s + 2), e3 = byte(4 * s + 3);
            mfma(s, v4i{(int)e0.x, (int)e1.x, (int)e2.x, (int)e3.x});
            B6[s] = (int)tern_bfi4(e0.y, e1.y, e2.y, e3.y);
          }
          mfma(6, B6);
          {
            uint2 e[10];
#pragma unroll
            for (int i = 0; i < 10; ++i) e[i] = byte(16 + i);
#pragma unroll
            for (int s = 4; s < 6; ++s) {
              const int b0 = 4 * (s - 4);
              mfma(s, v4i{(int)e[b0].x, (int)e[b0 + 1].x, (int)e[b0 + 2].x, (int)e[b0 + 3].x});
            }
            mfma(7, v4i{(int)tern_bfi4(e[0].y, e[1].y, e[2].y, e[3].y),
                        (int)tern_bfi4(e[4].y, e[5].y, e[6].y, e[7].y), (int)e[8].x, (int)e[9].x});
          }
        }
        // the block's scale (none past the row's last block)
        float d = tm::half(scl[(t * 16 + j) * nb + 4 * r + lg]);
        if (4 * r + 4 > nb && lg >= nb - 4 * r) d = 0.f;
        // the four limb sums as two exact pairs (|.| < 2^23):
        // sum_t D_t 2^(E - 6 - 7t) = (128 D_0 + D_1) 2^(E - 13) + (128 D_2 + D_3) 2^(E - 27)
        const int H = (acc[0] << 7) + acc[1], L = (acc[2] << 7) + acc[3];
        part[(r * ct + t) * 64 + lane] = ((float)H * sH + (float)L * sL) * d;
        if (++t == ct) { t = 0; ++r; }
        }
        load(c0, lt, lr, slot[u], z + D < n);   // the slot is free: the item D ahead
        if (++lt == ct) { lt = 0; ++lr; }
      }
    }
    __syncthreads();
    // ---- the chunk's tiles: rounds in order, then the four lane groups
    for (int tt = wave; tt < ct; tt += NWV) {
      float v = 0.f;
      for (int rr = 0; rr < nr; ++rr) v += part[(rr * ct + tt) * 64 + lane];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      const int row = (bx + (c0 + tt) * G) * 16 + j;
      epi.out(lane, row, nonfinite ? __builtin_nanf("") : v, lane < 16 && row < g.N);
    }
  }
}

}  // namespace hs
