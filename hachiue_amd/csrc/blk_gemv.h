// The F32, Q4_0 and Q4_1 lm_head GEMVs on the vector units, as
// device-function bodies shared by the GEMV kernels (lmhead_kernels.hip) and
// the all-greedy GEMV that keeps its rows' argmax (sampler_kernels.hip): the
// kernels differ only in what happens to each row's result (the epilogue).
// The method is described at the top of lmhead_kernels.hip.
#pragma once
#include "sampler_internal.h"

#include <hip/hip_runtime.h>

namespace hs {

namespace vg {

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t wrsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint32_t ld32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// Reads are issued by a unit's load() into raw dwords and consumed by its
// dot(), so that a wave requests several rows before it waits for any.  The
// bytes come from a source addressed by tensor offset: the tensor itself
// (GSrc) or a wave's copy of a span of it in LDS (LSrc).
struct GSrc {
  rsrc_t r;
  __device__ __forceinline__ uint32_t dw(uint32_t off) const { return ld32(r, off); }
  // n dwords from the aligned base; reads past lastdw are clamped to it (no
  // read past a block)
  template <int N>
  __device__ __forceinline__ void dws(uint32_t base, uint32_t lastdw, uint32_t (&d)[N]) const {
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = ld32(r, min(base + 4u * i, lastdw));
  }
  __device__ __forceinline__ void q4(uint32_t off, uint32_t (&o)[4]) const {
    const auto t = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    o[0] = t[0]; o[1] = t[1]; o[2] = t[2]; o[3] = t[3];
  }
};
struct LSrc {
  const uint32_t *b;   // the wave's buffer: tensor bytes from a0 (16-byte aligned) on
  uint32_t a0;
  __device__ __forceinline__ uint32_t dw(uint32_t off) const { return b[(off - a0) >> 2]; }
  // the buffer holds a batch and its slack: no clamp is needed; one address,
  // the dwords at immediate offsets from it
  template <int N>
  __device__ __forceinline__ void dws(uint32_t base, uint32_t, uint32_t (&d)[N]) const {
    const uint32_t *p = b + ((base - a0) >> 2);
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = p[i];
  }
  __device__ __forceinline__ void q4(uint32_t off, uint32_t (&o)[4]) const {
    const uint4 t = *reinterpret_cast<const uint4 *>(b + ((off - a0) >> 2));
    o[0] = t.x; o[1] = t.y; o[2] = t.z; o[3] = t.w;
  }
};

// The aligned dwords holding the bytes [off, off + 4 NDW) of an even off,
// of which only the bytes up to `last` (off <= last < off + 4 NDW) are used:
// d[i] = dword at (off & ~3) + 4 i, with reads past the dword holding `last`
// clamped to it, so nothing is read beyond the block (the resource covers the
// tensor rounded up to whole dwords, and no read can reach a page past it).
template <int NDW>
struct Span {
  uint32_t d[NDW + 1];
  uint32_t sh;   // off & 3: 0 or 2
  template <typename S>
  __device__ __forceinline__ void load(const S &r, uint32_t off, uint32_t last) {
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

// sum_{i<4} x[i] * byte_i(w), added to acc.  The empty asm hides how w was
// masked, so that each byte becomes one v_cvt_f32_ubyte0 .. 3 instead of a
// bit-field extract and a conversion.
__device__ __forceinline__ float dot4u8(uint32_t w, const float *x, float acc) {
  asm("" : "+v"(w));
  acc = fmaf(x[0], (float)(w & 0xFFu), acc);   // v_cvt_f32_ubyte0 .. 3
  acc = fmaf(x[1], (float)((w >> 8) & 0xFFu), acc);
  acc = fmaf(x[2], (float)((w >> 16) & 0xFFu), acc);
  acc = fmaf(x[3], (float)(w >> 24), acc);
  return acc;
}

// Sum over aligned groups of `seg` lanes (a power of two, at most 64) by DPP
// moves, without LDS: quad swaps, row mirrors, then row broadcasts for 32 and
// 64.  The group's last lane holds its total.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float seg_sum(float x, int seg) {
  if (seg >= 2) x += dpp_mov<0xB1, 0xF>(x);    // quad_perm [1, 0, 3, 2]
  if (seg >= 4) x += dpp_mov<0x4E, 0xF>(x);    // quad_perm [2, 3, 0, 1]
  if (seg >= 8) x += dpp_mov<0x141, 0xF>(x);   // row_half_mirror
  if (seg >= 16) x += dpp_mov<0x140, 0xF>(x);  // row_mirror
  if (seg >= 32) x += dpp_mov<0x142, 0xA>(x);  // row_bcast:15 into rows 1 and 3
  if (seg >= 64) x += dpp_mov<0x143, 0x8>(x);  // row_bcast:31 into row 3
  return x;
}

// ---- per-format unit geometry, reads and dot products ------------------------

template <int FMT> struct Unit;

// F32: unit j = weights [32 j, 32 j + 32), 128 bytes.
template <> struct Unit<kW_F32> {
  static constexpr int W = 32;
  struct Raw { uint32_t w[8][4]; };
  static __device__ __forceinline__ int xidx(int j, int i) { return 32 * j + i; }
  static __device__ __forceinline__ void sums(const float *, float *) {}
  template <typename S>
  static __device__ __forceinline__ void load(const S &r, uint32_t rb, int j, Raw &a) {
#pragma unroll
    for (int v = 0; v < 8; ++v) r.q4(rb + 128u * j + 16u * v, a.w[v]);
  }
  static __device__ __forceinline__ float dot(const Raw &a, int, const float *x, const float *) {
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < 8; ++v)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = fmaf(x[4 * v + q], __uint_as_float(a.w[v][q]), acc);
    return acc;
  }
};

// Q4_0: unit j = block j: d (fp16), 16 bytes of nibbles; w = (q - 8) d, low
// nibbles are weights 0..15, high 16..31.
template <> struct Unit<kW_Q4_0> {
  static constexpr int W = 32;
  struct Raw { Span<5> b; };
  static __device__ __forceinline__ int xidx(int j, int i) { return 32 * j + i; }
  static __device__ __forceinline__ void sums(const float *x, float *s) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
    s[0] = a;
  }
  template <typename S>
  static __device__ __forceinline__ void load(const S &r, uint32_t rb, int j, Raw &a) {
    a.b.load(r, rb + 18u * j, rb + 18u * j + 17u);
  }
  static __device__ __forceinline__ float dot(const Raw &a, int, const float *x, const float *s) {
    uint32_t b[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) b[i] = a.b.at(i);
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t q = __builtin_amdgcn_alignbyte(b[v + 1], b[v], 2);   // bytes 2 + 4v ..
      lo = dot4u8(q & 0x0F0F0F0Fu, x + 4 * v, lo);
      hi = dot4u8((q >> 4) & 0x0F0F0F0Fu, x + 16 + 4 * v, hi);
    }
    return h2f(b[0]) * ((lo + hi) - 8.f * s[0]);
  }
};

// Q4_1: unit j = block j: d, m (fp16), 16 bytes of nibbles; w = q d + m.
template <> struct Unit<kW_Q4_1> {
  static constexpr int W = 32;
  struct Raw { uint32_t b[5]; };
  static __device__ __forceinline__ int xidx(int j, int i) { return 32 * j + i; }
  static __device__ __forceinline__ void sums(const float *x, float *s) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
    s[0] = a;
  }
  template <typename S>
  static __device__ __forceinline__ void load(const S &r, uint32_t rb, int j, Raw &a) {
#pragma unroll
    for (int i = 0; i < 5; ++i) a.b[i] = r.dw(rb + 20u * j + 4u * i);
  }
  static __device__ __forceinline__ float dot(const Raw &a, int, const float *x, const float *s) {
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      lo = dot4u8(a.b[v + 1] & 0x0F0F0F0Fu, x + 4 * v, lo);
      hi = dot4u8((a.b[v + 1] >> 4) & 0x0F0F0F0Fu, x + 16 + 4 * v, hi);
    }
    return fmaf(h2f(a.b[0]), lo + hi, h2f(a.b[0] >> 16) * s[0]);
  }
};

}  // namespace vg

// One wave per group of rows; see the top of lmhead_kernels.hip.  NRU: units per lane
// (1: a row takes `seg` lanes; 2: a row takes all 64 lanes, units lane and
// lane + 64).  Each row's result goes to epi.out(lane, row, value, valid) from
// every lane (valid in the row's last lane), as the lanes reach it.
template <int FMT, int NRU, class Epi>
__device__ __forceinline__ void gemv_vec_body(const GemvArgs &g, Epi &epi) {
  using namespace vg;
  using U = Unit<FMT>;
  const int lane = threadIdx.x & 63;
  const int wave = (int)blockIdx.x * (kGemvThreads / 64) + (int)(threadIdx.x >> 6);
  const int nwaves = (int)gridDim.x * (kGemvThreads / 64);
  const int m = (int)blockIdx.y;
  const int seg = NRU == 1 ? g.seg : 64;
  const int slot = NRU == 1 ? lane / seg : 0;
  const int rows_per_step = 64 / seg;
  int unit[NRU];
  bool live[NRU];
#pragma unroll
  for (int u = 0; u < NRU; ++u) {
    unit[u] = NRU == 1 ? lane % seg : lane + 64 * u;
    live[u] = unit[u] < g.units;
  }
  // this lane's slice of x, in registers for every row
  float xr[NRU][U::W], xs[NRU][4];
  const float *xm = g.x + (int64_t)m * g.ldx;
#pragma unroll
  for (int u = 0; u < NRU; ++u) {
#pragma unroll
    for (int i = 0; i < U::W; ++i) xr[u][i] = live[u] ? xm[U::xidx(unit[u], i)] : 0.f;
    U::sums(xr[u], xs[u]);
  }
  const GSrc r{wrsrc(g.w, (g.w_bytes + 3u) & ~3u)};
  const int steps = (g.N + rows_per_step - 1) / rows_per_step;
  // two row steps per iteration: the reads of both are issued before either
  // is used (rows past N read nothing: their offsets lie past the resource)
  for (int st = wave; st < steps; st += 2 * nwaves) {
    const int n0 = st * rows_per_step + slot, n1 = n0 + nwaves * rows_per_step;
    typename U::Raw raw[2][NRU];
#pragma unroll
    for (int u = 0; u < NRU; ++u) {
      U::load(r, (uint32_t)n0 * g.row_bytes, unit[u], raw[0][u]);
      U::load(r, (uint32_t)n1 * g.row_bytes, unit[u], raw[1][u]);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < NRU; ++u)
        if (live[u]) acc += U::dot(raw[k][u], unit[u], xr[u], xs[u]);
      acc = seg_sum(acc, seg);
      const int n = k ? n1 : n0;
      epi.out(lane, n, acc, lane % seg == seg - 1 && n < g.N);
    }
  }
}

// The block formats through LDS (the LDS at glds: gemv_lds_bytes(FMT)).
// Their blocks are 2-byte aligned (Q4_0,
// Q6_K) or smaller than a lane's reads, so per-lane reads of the tensor touch
// a different cache line in every lane.  Instead each wave reads the
// contiguous bytes of a batch of rows (gemv_batch_steps() row steps) with
// 16-byte loads, consecutive lanes on consecutive bytes, into its own LDS
// buffer; the lanes then take their units from there.  The next batch's
// reads are in flight (in registers) while a batch is taken apart.
template <int FMT, int NRU, class Epi>
__device__ __forceinline__ void gemv_lds_body(const GemvArgs &g, uint4 *glds, Epi &epi) {
  using namespace vg;
  using U = Unit<FMT>;
  constexpr int CH = gemv_batch_chunks(FMT);   // 16-byte reads per lane and batch
  constexpr int SB = gemv_batch_steps(FMT) / NRU;
  const int lane = threadIdx.x & 63;
  uint4 *buf = glds + (threadIdx.x >> 6) * (64 * CH);
  const int wave = (int)blockIdx.x * (kGemvThreads / 64) + (int)(threadIdx.x >> 6);
  const int nwaves = (int)gridDim.x * (kGemvThreads / 64);
  const int m = (int)blockIdx.y;
  const int seg = NRU == 1 ? g.seg : 64;
  const int slot = NRU == 1 ? lane / seg : 0;
  const int rows_per_step = 64 / seg;
  int unit[NRU];
  bool live[NRU];
#pragma unroll
  for (int u = 0; u < NRU; ++u) {
    unit[u] = NRU == 1 ? lane % seg : lane + 64 * u;
    live[u] = unit[u] < g.units;
  }
  float xr[NRU][U::W], xs[NRU][4];
  const float *xm = g.x + (int64_t)m * g.ldx;
#pragma unroll
  for (int u = 0; u < NRU; ++u) {
#pragma unroll
    for (int i = 0; i < U::W; ++i) xr[u][i] = live[u] ? xm[U::xidx(unit[u], i)] : 0.f;
    U::sums(xr[u], xs[u]);
  }
  // A 16-byte read at or past the resource's end returns zeros; the resource
  // covers the tensor rounded up to 16 bytes, so the last read stays within
  // the 16-byte line of the tensor's last byte.
  const rsrc_t r = wrsrc(g.w, (g.w_bytes + 15u) & ~15u);
  const int rpb = SB * rows_per_step;
  const int batches = (g.N + rpb - 1) / rpb;
  uint32_t pf[CH][4];
  uint32_t a0n = 0;
  int nchn = 0;
  auto fetch = [&](int b) {   // batch b's bytes into pf
    const int r0 = b * rpb, r1 = min(g.N, r0 + rpb);
    const uint32_t s0 = (uint32_t)r0 * g.row_bytes, s1 = (uint32_t)r1 * g.row_bytes;
    a0n = s0 & ~15u;
    nchn = (int)((s1 - a0n + 15u) >> 4);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      const auto t = __builtin_amdgcn_raw_buffer_load_b128(r, c < nchn ? a0n + 16u * c : 0xFFFFFFF0u,
                                                           0, 0);
      pf[i][0] = t[0]; pf[i][1] = t[1]; pf[i][2] = t[2]; pf[i][3] = t[3];
    }
  };
  int b = wave;
  if (b < batches) fetch(b);
  while (b < batches) {
    const uint32_t a0 = a0n;
    const int nch = nchn;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) buf[c] = make_uint4(pf[i][0], pf[i][1], pf[i][2], pf[i][3]);
    }
    const int nb = b + nwaves;
    if (nb < batches) fetch(nb);
    const LSrc src{reinterpret_cast<const uint32_t *>(buf), a0};
    // every step's unit bytes first, then the dot products: the LDS reads
    // of a batch are in flight together
    typename U::Raw rw[SB][NRU];
#pragma unroll
    for (int k = 0; k < SB; ++k) {
      const int n = (b * SB + k) * rows_per_step + slot;
#pragma unroll
      for (int u = 0; u < NRU; ++u) U::load(src, (uint32_t)n * g.row_bytes, unit[u], rw[k][u]);
    }
#pragma unroll
    for (int k = 0; k < SB; ++k) {
      const int n = (b * SB + k) * rows_per_step + slot;
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < NRU; ++u) {
        if (live[u]) acc += U::dot(rw[k][u], unit[u], xr[u], xs[u]);
      }
      acc = seg_sum(acc, seg);
      epi.out(lane, n, acc, lane % seg == seg - 1 && n < g.N);
    }
    b = nb;
  }
}

}  // namespace hs
