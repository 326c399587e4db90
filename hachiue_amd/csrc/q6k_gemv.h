// The Q6_K lm_head GEMV on the matrix cores, as a device-function body
// shared by the GEMV kernel (lmhead_kernels.hip) and the GEMV that samples
// its own rows (sampler_kernels.hip): the kernels differ only in what
// happens to each tile's results (the epilogue).
#pragma once
#include "sampler_internal.h"

#include <hip/hip_runtime.h>

namespace hs {

// ---- Q6_K on the matrix cores
//
// A Q6_K weight is d * sc * (q - 32) with q a 6-bit integer.  x is held as
// four int8 limbs per scale group of 16 positions: with 2^E above the group's
// largest |x|, a_t = rint(r_{t-1} * 2^(6 + 7t - E)) and r_t the exact
// remainder, so |a_t| <= 64 and x - sum_t a_t 2^(E - 6 - 7t) is below
// 2^(E - 28) (binary32 sums of the products would round at 2^-24 of each
// term).  v_mfma_i32_16x16x64_i8 then forms exact integer dot products: B
// (64 x 16) holds the q bytes of 16 rows, lane (j, G) the 16 positions of
// scale group G of row j; A (16 x 64) holds in row 4G + t limb t of that
// group's x, zero elsewhere, so the result's lane (j, G) receives the four
// limb sums of its own (row, group), D[4G + t][j].  The -32 enters as an
// integer (D - 32 sum_b a_t), and the row's sum is
// d * sum over groups of sc * sum_t 2^(E - 6 - 7t) (D_t - 32 A_t).
//
// Work: a wave takes tiles of 16 consecutive rows; a tile's super-blocks go
// through LDS two at a time ("slabs": 16 rows x 448 bytes, the 16-byte
// aligned cover of each row's two super-blocks), read straight into LDS by
// buffer_load ... lds into a ring of NB buffers per wave: NB - 1 slabs are
// in flight while one is taken apart (one wave per SIMD, LDS-bound; the
// bytes in flight per CU are what keep HBM busy).
// q bytes of a lane: half n = G / 2, positions 16 h .. 16 h + 15 (h = G % 2)
// of quarter qq, from ql (low nibbles for quarters 0 and 1, high for 2 and
// 3) and qh (bits 2 qq): weight 128 n + 32 qq + l of a super-block has its
// low bits in ql byte 64 n + 32 (qq & 1) + l and its high bits in qh byte
// 32 n + l; scale 8 n + h + 2 qq (src/gguf.ts:206-232).
namespace q6m {
constexpr int kSB = 1;                               // super-blocks per slab
constexpr int kNB = 2;                               // ring depth (slabs per wave)
constexpr int kRowChunks = (210 * kSB + 14 + 15) / 16;   // 16-byte chunks per row: 14
constexpr int kSlabRowBytes = 16 * kRowChunks;       // 224
constexpr int kLoads = (16 * kRowChunks + 63) / 64;  // 1 KiB loads per slab: 4, the last
constexpr int kLastLanes = 16 * kRowChunks - 64 * (kLoads - 1);   //   by 32 lanes
constexpr int kSlabBytes = 16 * 16 * kRowChunks;     // 3584
constexpr int kWaves = 8;                            // per workgroup, 2 workgroups per CU
constexpr int kThreads = 64 * kWaves;
typedef int v4i __attribute__((ext_vector_type(4)));
// LDS bytes of a slab addressed by tensor offset, the aligned dwords of a
// byte span, and binary16 scales: the Q6_K body's own copies of the block
// formats' helpers.
struct LSrc {
  const uint32_t *b;   // tensor bytes from a0 (16-byte aligned) on
  uint32_t a0;
  __device__ __forceinline__ uint32_t dw(uint32_t off) const { return b[(off - a0) >> 2]; }
  template <int N>
  __device__ __forceinline__ void dws(uint32_t base, uint32_t, uint32_t (&d)[N]) const {
    const uint32_t *p = b + ((base - a0) >> 2);
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = p[i];
  }
};
// the aligned dwords holding the bytes [off, off + 4 NDW) of an even off
template <int NDW>
struct Span {
  uint32_t d[NDW + 1];
  uint32_t sh;   // off & 3: 0 or 2
  __device__ __forceinline__ void load(const LSrc &r, uint32_t off, uint32_t last) {
    sh = off & 3u;
    r.dws(off & ~3u, last & ~3u, d);
  }
  // bytes [off + 4 i, off + 4 i + 4)
  __device__ __forceinline__ uint32_t at(int i) const {
    return __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
  }
};
__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}
}  // namespace q6m

__host__ __device__ inline size_t gemv_q6k_mfma_lds_bytes(int K) {
  // A operands: 256 B per 64 positions; per scale group 32 A_t (int4) and
  // 2^(E - 6 - 7t) (float4); the slab rings
  return (size_t)(K / 64) * 256 + (size_t)(K / 16) * 32 +
         (size_t)q6m::kWaves * q6m::kNB * q6m::kSlabBytes;
}

// The body of a kernel of 2 workgroups per CU (16 waves: at most 128 VGPRs)
// and q6m::kThreads threads: activation row blockIdx.y, its LDS at `lds`
// (gemv_q6k_mfma_lds_bytes(K)).  Each row's result goes to
// epi.out(lane, row, value, valid), called by every lane of a wave at once,
// lanes 0..15 holding the 16 rows of a tile (valid: lane < 16, row < N).
template <class Epi>
__device__ __forceinline__ void q6k_gemv_body(const GemvArgs &g, uint8_t *lds, Epi &epi) {
  constexpr int NB = q6m::kNB;
  using namespace q6m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = (int)blockIdx.y;
  const int K = g.K, NG = K / 16, NS = K / 256;
  v4i *aop = reinterpret_cast<v4i *>(lds);                        // [K/64][4 G][4 t]
  v4i *p32 = reinterpret_cast<v4i *>(lds + (size_t)(K / 64) * 256);
  float4 *psc = reinterpret_cast<float4 *>(p32 + NG);
  uint8_t *ring = reinterpret_cast<uint8_t *>(psc + NG) + (size_t)wave * NB * kSlabBytes;


  // Work: the waves take whole tiles round-robin for as many full rounds as
  // there are; the tiles left (fewer than the waves) are cut into P slab
  // ranges each, so that every wave ends within about a slab of the others.
  // A cut tile's parts hand their partial sums over: each publishes its 16
  // sums, then counts itself in; the part that counts P adds the P sums in
  // part order (the result does not depend on which part came last) and
  // writes y.
  const int nw = (int)gridDim.x * q6m::kWaves;
  const int wg = (int)blockIdx.x * q6m::kWaves + wave;
  const int ntiles = (g.N + 15) >> 4;
  const int nsl = (NS + kSB - 1) / kSB;
  const int rfull = ntiles / nw, tail = ntiles - rfull * nw;
  int P = tail > 0 ? nw / tail : 1;
  P = P < nsl ? P : nsl;
  const bool has_part = tail > 0 && wg < tail * P;
  const int ptt = wg / P, pidx = wg - ptt * P;           // tail tile index, part
  const int p0 = pidx * nsl / P, p1 = (pidx + 1) * nsl / P;
  const int items = rfull * nsl + (has_part ? p1 - p0 : 0);
  // item z: its tile, its slab, and whether it ends a segment
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
  const int j = lane & 15, G = lane >> 4, n = G >> 1, h = G & 1;
  // this lane's A operand row: A row (lane & 15) is limb (lane & 3) of lane
  // group (lane & 15) >> 2, non-zero only in that lane group
  const bool a_live = ((lane & 15) >> 2) == G;

  // The reads into LDS are issued from inline assembly, so that the compiler
  // does not make every LDS read wait for them (it cannot tell the ring's
  // buffers apart); the waits below are explicit.  The compiler's own waits
  // for its vector memory operations stay correct: extra operations in
  // flight only make them wait longer.
  const uint64_t wbase = reinterpret_cast<uint64_t>(g.w);
  const v4i rs = v4i{(int)(uint32_t)wbase, (int)(uint32_t)(wbase >> 32),
                     (int)((g.w_bytes + 15u) & ~15u), 0x00020000};
  auto issue = [&](int z, uint8_t *dst) {   // slab z of this wave into dst
    int tile, sl;
    (void)item(z, tile, sl);
    const int s0 = kSB * sl;
#pragma unroll
    for (int c = 0; c < kLoads; ++c) {
      const int q = c * 64 + lane, rj = q / kRowChunks, cc = q % kRowChunks;
      const int row = tile * 16 + rj;
      const uint32_t gs = (uint32_t)row * RB + 210u * (uint32_t)s0;
      const uint32_t off = row < g.N ? (gs & ~15u) + 16u * (uint32_t)cc : 0xFFFFFFF0u;
      const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) uint8_t *)(dst + c * 1024)));
      // the last load's lanes past the slab are masked off: they write no LDS
      // (M0 is the compiler's: it is saved and restored around the load)
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
  // (whose limbs are undefined) makes the row's results NaN
  __shared__ int nonfin;
  if (tid == 0) nonfin = 0;
  __syncthreads();
  const float *xm = g.x + (int64_t)m * g.ldx;
  for (int gi = tid; gi < NG; gi += q6m::kThreads) {
    float xv[16], mx = 0.f;
    bool fin = true;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      xv[b] = xm[16 * gi + b];
      mx = fmaxf(mx, fabsf(xv[b]));
      fin = fin && __builtin_isfinite(xv[b]);
    }
    if (!fin) nonfin = 1;
    int E = 0;
    (void)frexpf(mx, &E);   // mx < 2^E
    uint32_t limb[4][4];
    int At[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      At[t] = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) limb[t][w] = 0u;
    }
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      float r = xv[b];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float a = rintf(ldexpf(r, 6 + 7 * t - E));
        r -= ldexpf(a, E - 6 - 7 * t);   // exact: a 2^(E-6-7t) is within half a step of r
        const int ai = (int)a;
        At[t] += ai;
        limb[t][b >> 2] |= ((uint32_t)ai & 0xFFu) << (8 * (b & 3));
      }
    }
    // group gi = 16 s + 8 n + 2 qq + h: MFMA 4 s + qq, lane group G = 2 n + h
    const int sb = gi >> 4, n = (gi >> 3) & 1, qq = (gi >> 1) & 3, h = gi & 1;
    const int mi = 4 * sb + qq, G = 2 * n + h;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      aop[(mi * 4 + G) * 4 + t] = v4i{(int)limb[t][0], (int)limb[t][1], (int)limb[t][2], (int)limb[t][3]};
    p32[gi] = v4i{32 * At[0], 32 * At[1], 32 * At[2], 32 * At[3]};
    psc[gi] = make_float4(ldexpf(1.f, E - 6), ldexpf(1.f, E - 13), ldexpf(1.f, E - 20),
                          ldexpf(1.f, E - 27));
  }
  __syncthreads();
  const bool nan_out = nonfin != 0;
  for (int z = 0; z < items; ++z) {
    const uint8_t *cur = ring + (z % NB) * kSlabBytes;
    if (z + NB - 1 < items) {
      // its buffer was taken apart in the previous step: those reads are done
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
      issue(z + NB - 1, ring + ((z + NB - 1) % NB) * kSlabBytes);
    }
    // slab z has arrived once at most the later slab's loads are in flight
    // (kLoads); a y store among them only makes the wait longer
    static_assert(NB == 2 && kLoads < 16, "one later slab, vmcnt below 16");
    if (z + 1 < items)
      __builtin_amdgcn_s_waitcnt(0x0F70 | kLoads);   // vmcnt(kLoads)
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);            // vmcnt(0)
    asm volatile("" ::: "memory");
    int tile, sl;
    const bool seg_end = item(z, tile, sl);
    const int s0 = kSB * sl;
    const int ns = NS - s0 < kSB ? NS - s0 : kSB;
    const int row = tile * 16 + j;
    const uint32_t sh = ((uint32_t)row * RB + 210u * (uint32_t)s0) & 15u;
    const q6m::LSrc src{reinterpret_cast<const uint32_t *>(cur + j * kSlabRowBytes), 0u};
    for (int u = 0; u < ns; ++u) {
      const int sbk = s0 + u;
      const uint32_t o = sh + 210u * (uint32_t)u;
      const uint32_t oa = o + 64u * n + 16u * h, ob = oa + 32u, oh = o + 128u + 32u * n + 16u * h;
      const uint32_t os = o + 192u + 8u * n, od = o + 208u;
      q6m::Span<4> qa, qb, qh;
      q6m::Span<2> sc;
      qa.load(src, oa, oa + 15u);
      qb.load(src, ob, ob + 15u);
      qh.load(src, oh, oh + 15u);
      sc.load(src, os, os + 7u);
      const uint32_t dd = src.dw(od & ~3u) >> (8u * (od & 3u));
      v4i bq[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t a = qa.at(w), b = qb.at(w), hv = qh.at(w);
        bq[0][w] = (int)((a & 0x0F0F0F0Fu) | ((hv << 4) & 0x30303030u));
        bq[1][w] = (int)((b & 0x0F0F0F0Fu) | ((hv << 2) & 0x30303030u));
        bq[2][w] = (int)(((a >> 4) & 0x0F0F0F0Fu) | (hv & 0x30303030u));
        bq[3][w] = (int)(((b >> 4) & 0x0F0F0F0Fu) | ((hv >> 2) & 0x30303030u));
      }
      float accsb = 0.f;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int mi = 4 * sbk + qq;
        const v4i al = aop[(mi * 4 + G) * 4 + (lane & 3)];
        const v4i a = a_live ? al : v4i{0, 0, 0, 0};
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bq[qq], v4i{0, 0, 0, 0}, 0, 0, 0);
        const int gi = 16 * sbk + 8 * n + 2 * qq + h;
        const v4i pa = p32[gi];
        const float4 ps = psc[gi];
        float val = (float)(d[0] - pa[0]) * ps.x;
        val = fmaf((float)(d[1] - pa[1]), ps.y, val);
        val = fmaf((float)(d[2] - pa[2]), ps.z, val);
        val = fmaf((float)(d[3] - pa[3]), ps.w, val);
        const uint32_t scb = (sc.at(qq >> 1) >> (8u * (uint32_t)(h + 2 * (qq & 1)))) & 0xFFu;
        accsb = fmaf((float)(int8_t)scb, val, accsb);
      }
      acc = fmaf(q6m::h2f(dd), accsb, acc);
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
