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
// Q6_K runs on the matrix cores (gemv_q6k_mfma_kernel, described there).  The
// other formats use the vector units, one wave per group of rows:
//   every lane owns a fixed "unit" of each row: 32 weights (F32, Q4_0, Q4_1,
//   Q4_K: half of a 32-byte quant pair).  Its slice of x stays in registers
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
#include "tern_gemv.h"

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

namespace hs {

namespace {

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

// Q4_K: super-block s = j / 8 (header: d, dmin, 12 bytes of 6-bit scales and
// mins; 128 bytes of nibbles), part t = j % 8: the 16 bytes
// 16 + 32 (t / 2) + 16 (t % 2) of the nibbles.  Their low nibbles are
// weights 64 p + 16 h + i of sub-block 2 p, the high ones 64 p + 32 + 16 h + i
// of sub-block 2 p + 1 (p = t / 2, h = t % 2, i < 16);
// w = d sc q - dmin mn.
template <> struct Unit<kW_Q4_K> {
  static constexpr int W = 32;
  struct Raw { uint32_t hd[4], q[4]; };
  static __device__ __forceinline__ int xidx(int j, int i) {
    const int s = j >> 3, t = j & 7, p = t >> 1, h = t & 1;
    return 256 * s + 64 * p + 16 * h + (i < 16 ? i : 16 + i);
  }
  static __device__ __forceinline__ void sums(const float *x, float *s) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { a += x[i]; b += x[16 + i]; }
    s[0] = a;
    s[1] = b;
  }
  template <typename S>
  static __device__ __forceinline__ void load(const S &r, uint32_t rb, int j, Raw &a) {
    const int sb = j >> 3, t = j & 7, p = t >> 1, h = t & 1;
    const uint32_t o = rb + 144u * sb;
    r.q4(o, a.hd);
    r.q4(o + 16u + 32u * p + 16u * h, a.q);
  }
  static __device__ __forceinline__ float dot(const Raw &a, int j, const float *x, const float *s) {
    const int p = (j & 7) >> 1;
    // 6-bit scale / min of sub-block k (src/gguf.ts:178-186).  Header bytes
    // 4..7, 8..11, 12..15 are hd[1], hd[2], hd[3]; byte k & 3 of each is
    // taken with a shift, so no register is indexed at run time.
    auto scmin = [&](int k, float &sc, float &mn) {
      const uint32_t sh = 8u * (uint32_t)(k & 3);
      const uint32_t b1 = a.hd[1] >> sh, b2 = a.hd[2] >> sh, b3 = a.hd[3] >> sh;
      const uint32_t u = k < 4 ? (b1 & 63u) : ((b3 & 15u) | (((b1 >> 6) & 3u) << 4));
      const uint32_t c = k < 4 ? (b2 & 63u) : (((b3 >> 4) & 15u) | (((b2 >> 6) & 3u) << 4));
      sc = (float)u;
      mn = (float)c;
    };
    float sc0, mn0, sc1, mn1;
    scmin(2 * p, sc0, mn0);
    scmin(2 * p + 1, sc1, mn1);
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      lo = dot4u8(a.q[v] & 0x0F0F0F0Fu, x + 4 * v, lo);
      hi = dot4u8((a.q[v] >> 4) & 0x0F0F0F0Fu, x + 16 + 4 * v, hi);
    }
    const float d = h2f(a.hd[0]), dmin = h2f(a.hd[0] >> 16);
    return d * fmaf(sc0, lo, sc1 * hi) - dmin * fmaf(mn0, s[0], mn1 * s[1]);
  }
};

}  // namespace

// One wave per group of rows; see the top of the file.  NRU: units per lane
// (1: a row takes `seg` lanes; 2: a row takes all 64 lanes, units lane and
// lane + 64).
template <int FMT, int NRU>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs g) {
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
      if (lane % seg == seg - 1 && n < g.N) g.y[(int64_t)m * g.ldy + n] = acc;
    }
  }
}

// The block formats through LDS.  Their blocks are 2-byte aligned (Q4_0,
// Q6_K) or smaller than a lane's reads, so per-lane reads of the tensor touch
// a different cache line in every lane.  Instead each wave reads the
// contiguous bytes of a batch of rows (gemv_batch_steps() row steps) with
// 16-byte loads, consecutive lanes on consecutive bytes, into its own LDS
// buffer; the lanes then take their units from there.  The next batch's
// reads are in flight (in registers) while a batch is taken apart.
template <int FMT, int NRU>
__global__ __launch_bounds__(kGemvThreads) void gemv_lds_kernel(GemvArgs g) {
  using U = Unit<FMT>;
  constexpr int CH = gemv_batch_chunks(FMT);   // 16-byte reads per lane and batch
  constexpr int SB = gemv_batch_steps(FMT) / NRU;
  extern __shared__ uint4 glds[];
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
      if (lane % seg == seg - 1 && n < g.N) g.y[(int64_t)m * g.ldy + n] = acc;
    }
    b = nb;
  }
}

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
}  // namespace q6m

size_t gemv_q6k_mfma_lds_bytes(int K) {
  // A operands: 256 B per 64 positions; per scale group 32 A_t (int4) and
  // 2^(E - 6 - 7t) (float4); the slab rings
  return (size_t)(K / 64) * 256 + (size_t)(K / 16) * 32 +
         (size_t)q6m::kWaves * q6m::kNB * q6m::kSlabBytes;
}

// 2 workgroups per CU (16 waves): at most 128 VGPRs
__global__ __launch_bounds__(q6m::kThreads, 2) void gemv_q6k_mfma_kernel(GemvArgs g) {
  constexpr int NB = q6m::kNB;
  using namespace q6m;
  extern __shared__ uint4 qlds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = (int)blockIdx.y;
  const int K = g.K, NG = K / 16, NS = K / 256;
  uint8_t *lds = reinterpret_cast<uint8_t *>(qlds);
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
    const LSrc src{reinterpret_cast<const uint32_t *>(cur + j * kSlabRowBytes), 0u};
    for (int u = 0; u < ns; ++u) {
      const int sbk = s0 + u;
      const uint32_t o = sh + 210u * (uint32_t)u;
      const uint32_t oa = o + 64u * n + 16u * h, ob = oa + 32u, oh = o + 128u + 32u * n + 16u * h;
      const uint32_t os = o + 192u + 8u * n, od = o + 208u;
      Span<4> qa, qb, qh;
      Span<2> sc;
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
      acc = fmaf(h2f(dd), accsb, acc);
    }
    if (seg_end) {   // the four lane groups of a row add up
      acc += __shfl_xor(acc, 16);
      acc += __shfl_xor(acc, 32);
      if (z < rfull * nsl || P == 1) {
        if (lane < 16 && row < g.N) g.y[(int64_t)m * g.ldy + row] = nan_out ? __builtin_nanf("") : acc;
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
          if (lane < 16 && row < g.N)
            g.y[(int64_t)m * g.ldy + row] = nan_out ? __builtin_nanf("") : sum;
          if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      acc = 0.f;
    }
  }
}

// ---- Q1_0 / PQ2_0 / PTQ1_0 on the matrix cores (the body: tern_gemv.h)


namespace {
// Each tile's results straight to y.
struct StoreY {
  float *y;
  __device__ __forceinline__ void out(int, int row, float v, bool valid) {
    if (valid) y[row] = v;
  }
};
}  // namespace

template <int FMT>
__global__ __launch_bounds__(64 * tm::waves<FMT>()) void gemv_tern_kernel(GemvArgs g) {
  extern __shared__ uint4 tlds[];
  StoreY epi{g.y + (int64_t)blockIdx.y * g.ldy};
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

hipError_t launch_q6k_mfma(GemvArgs g, hipStream_t stream, hipEvent_t *ev, hipEvent_t done) {
  const size_t lds = gemv_q6k_mfma_lds_bytes(g.K);
  const int ntiles = (g.N + 15) / 16;
  const int res = resident_blocks(reinterpret_cast<const void *>(gemv_q6k_mfma_kernel), (uint32_t)lds,
                                  q6m::kThreads);
  int blocks = (ntiles + q6m::kWaves - 1) / q6m::kWaves;
  blocks = blocks < res ? blocks : res;
  // every wave of an activation row owns a hand-over slot
  blocks = blocks < g.part_cap / q6m::kWaves ? blocks : g.part_cap / q6m::kWaves;
  if (blocks < 1 || !g.part || !g.tile_cnt) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)g.M), block(q6m::kThreads);
  if (ev)
    hipExtLaunchKernelGGL(gemv_q6k_mfma_kernel, grid, block, lds, stream, ev[0], ev[1], 0u, g);
  else if (done)
    hipExtLaunchKernelGGL(gemv_q6k_mfma_kernel, grid, block, lds, stream, nullptr, done, 0u, g);
  else
    hipLaunchKernelGGL(gemv_q6k_mfma_kernel, grid, block, lds, stream, g);
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
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(gemv_q6k_mfma_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)gemv_q6k_mfma_lds_bytes(kGemvMaxK));
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
    case kW_Q4_K: return two ? launch_fmt<kW_Q4_K, 2>(g, stream, ev, done) : launch_fmt<kW_Q4_K, 1>(g, stream, ev, done);
    case kW_Q6_K: return launch_q6k_mfma(g, stream, ev, done);
    case kW_Q1_0: return launch_tern<kW_Q1_0>(g, stream, ev, done);
    case kW_PQ2_0: return launch_tern<kW_PQ2_0>(g, stream, ev, done);
    case kW_PTQ1_0: return launch_tern<kW_PTQ1_0>(g, stream, ev, done);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hs
