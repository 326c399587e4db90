/*
 * CPU restatement of hachiue's lm_head GEMV.  TEST INFRASTRUCTURE ONLY (see
 * lmhead_oracle.h).
 */
#include "lmhead_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int orc_block_weights(int type) {
  switch (type) {
    case ORC_W_F32: return 1;
    case ORC_W_Q4_0: case ORC_W_Q4_1: return 32;
    case ORC_W_Q4_K: case ORC_W_Q6_K: return 256;
    case ORC_W_Q1_0: case ORC_W_PQ2_0: case ORC_W_PTQ1_0: return 128;
    default: return 0;
  }
}

int orc_block_bytes(int type) {
  switch (type) {
    case ORC_W_F32: return 4;
    case ORC_W_Q4_0: return 18;
    case ORC_W_Q4_1: return 20;
    case ORC_W_Q4_K: return 144;
    case ORC_W_Q6_K: return 210;
    case ORC_W_Q1_0: return 18;    /* 2 B binary16 scale + 16 B sign bits */
    case ORC_W_PQ2_0: return 34;   /* 2 B scale + 32 B 2-bit codes */
    case ORC_W_PTQ1_0: return 28;  /* 24 B qs + 2 B qh (base-3 trits) + 2 B scale */
    default: return 0;
  }
}

/* src/gguf.ts:81-88 */
float orc_fp16(uint16_t h) {
  const double s = (h & 0x8000) ? -1.0 : 1.0;   /* a JS number: -1 * 0 is -0 */
  const int e = (h >> 10) & 0x1f;
  const int m = h & 0x03ff;
  if (e == 0) return (float)(s * m * ldexp(1.0, -24));
  if (e == 31) return m ? NAN : (float)(s * INFINITY);
  return (float)(s * (1024 + m) * ldexp(1.0, e - 25));
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q4_K 6-bit scale and min of 32-weight sub-block j (src/gguf.ts:178-186). */
static void q4k_scale_min(const uint8_t *blk, int j, int *sc, int *mn) {
  if (j < 4) {
    *sc = blk[4 + j] & 63;
    *mn = blk[8 + j] & 63;
  } else {
    *sc = (blk[8 + j] & 0x0f) | ((blk[j] >> 6) << 4);
    *mn = (blk[8 + j] >> 4) | ((blk[4 + j] >> 6) << 4);
  }
}

/* Q6_K quant (-32 .. 31) and scale index of weight i of a super-block
 * (src/gguf.ts:206-232). */
static void q6k_weight(const uint8_t *blk, int i, int *q, int *sidx) {
  const int n = i / 128, r = i % 128, qq = r / 32, l = r % 32;
  const uint8_t ql = blk[n * 64 + (qq & 1) * 32 + l];
  const uint8_t qh = blk[128 + n * 32 + l];
  const int lo = qq < 2 ? (ql & 0x0f) : (ql >> 4);
  *q = (lo | (((qh >> (2 * qq)) & 3) << 4)) - 32;
  *sidx = n * 8 + (l >> 4) + 2 * qq;
}

/* Code c (0, 1 or 2) of weight j of a PTQ1_0 block, and the PTQ1_0 trit of
 * byte b (src/gguf.ts:111-144): bytes 0..15 hold weights m + 16 n, bytes
 * 16..23 weights 80 + m + 8 n (n = 0..4), bytes 24..25 weights 120 + h + 2 n
 * (n = 0..3); trit n of byte b is ((b * 3^n mod 256) * 3) >> 8. */
static int ptq1_trit(uint8_t b, int n) {
  static const int pow3[5] = {1, 3, 9, 27, 81};
  return (((b * pow3[n]) & 0xff) * 3) >> 8;
}
static int ptq1_code(const uint8_t *blk, int j) {
  if (j < 80) return ptq1_trit(blk[j % 16], j / 16);
  if (j < 120) return ptq1_trit(blk[16 + (j - 80) % 8], (j - 80) / 8);
  return ptq1_trit(blk[24 + (j - 120) % 2], (j - 120) / 2);
}

/* Signed multiple of the block scale of weight j of a Q1_0 / PQ2_0 / PTQ1_0
 * block (src/gguf.ts:95-144): Q1_0 bit ? 1 : -1, PQ2_0 q - 1, PTQ1_0 c - 1. */
static int tern_code(int type, const uint8_t *blk, int j) {
  if (type == ORC_W_Q1_0) return ((blk[2 + (j >> 3)] >> (j & 7)) & 1) ? 1 : -1;
  if (type == ORC_W_PQ2_0) return ((blk[2 + (j >> 2)] >> ((j & 3) * 2)) & 3) - 1;
  return ptq1_code(blk, j) - 1;
}
static uint16_t tern_scale(int type, const uint8_t *blk) {
  return type == ORC_W_PTQ1_0 ? rd16(blk + 26) : rd16(blk);
}

/* src/gguf.ts:149-230 and :93-147 */
int orc_dequant_row(int type, const uint8_t *row, int64_t K, float *out) {
  const int B = orc_block_weights(type), BB = orc_block_bytes(type);
  if (!B || K % B) return -1;
  for (int64_t b = 0; b < K / B; ++b) {
    const uint8_t *blk = row + b * BB;
    float *o = out + b * B;
    if (type == ORC_W_F32) {
      memcpy(o, blk, 4);
    } else if (type == ORC_W_Q4_0) {
      const float d = orc_fp16(rd16(blk));
      for (int j = 0; j < 16; ++j) {
        o[j] = (float)((blk[2 + j] & 0x0f) - 8) * d;
        o[16 + j] = (float)((blk[2 + j] >> 4) - 8) * d;
      }
    } else if (type == ORC_W_Q4_1) {
      const float d = orc_fp16(rd16(blk)), m = orc_fp16(rd16(blk + 2));
      for (int j = 0; j < 16; ++j) {
        o[j] = (float)(blk[4 + j] & 0x0f) * d + m;
        o[16 + j] = (float)(blk[4 + j] >> 4) * d + m;
      }
    } else if (type == ORC_W_Q4_K) {
      const float d = orc_fp16(rd16(blk)), dmin = orc_fp16(rd16(blk + 2));
      for (int p = 0; p < 4; ++p) {
        int s1, m1, s2, m2;
        q4k_scale_min(blk, 2 * p, &s1, &m1);
        q4k_scale_min(blk, 2 * p + 1, &s2, &m2);
        const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        const float d2 = d * (float)s2, mm2 = dmin * (float)m2;
        for (int l = 0; l < 32; ++l) {
          o[64 * p + l] = d1 * (float)(blk[16 + 32 * p + l] & 0x0f) - mm1;
          o[64 * p + 32 + l] = d2 * (float)(blk[16 + 32 * p + l] >> 4) - mm2;
        }
      }
    } else if (type == ORC_W_Q6_K) {
      const float d = orc_fp16(rd16(blk + 208));
      for (int i = 0; i < 256; ++i) {
        int q, si;
        q6k_weight(blk, i, &q, &si);
        o[i] = d * (float)(int8_t)blk[192 + si] * (float)q;
      }
    } else if (type == ORC_W_Q1_0 || type == ORC_W_PQ2_0 || type == ORC_W_PTQ1_0) {
      const double d = orc_fp16(tern_scale(type, blk));
      for (int j = 0; j < 128; ++j) o[j] = (float)(tern_code(type, blk, j) * d);
    } else {
      return -1;
    }
  }
  return 0;
}

/* Weight i of a row as an exact binary64 (every product of the format's
 * fields fits 53 bits). */
static double exact_weight(int type, const uint8_t *row, int64_t i) {
  const int B = orc_block_weights(type), BB = orc_block_bytes(type);
  const uint8_t *blk = row + (i / B) * BB;
  const int j = (int)(i % B);
  if (type == ORC_W_F32) {
    float f;
    memcpy(&f, blk, 4);
    return f;
  }
  if (type == ORC_W_Q4_0) {
    const int q = j < 16 ? (blk[2 + j] & 0x0f) : (blk[2 + j - 16] >> 4);
    return (double)orc_fp16(rd16(blk)) * (q - 8);
  }
  if (type == ORC_W_Q4_1) {
    const int q = j < 16 ? (blk[4 + j] & 0x0f) : (blk[4 + j - 16] >> 4);
    return (double)orc_fp16(rd16(blk)) * q + (double)orc_fp16(rd16(blk + 2));
  }
  if (type == ORC_W_Q1_0 || type == ORC_W_PQ2_0 || type == ORC_W_PTQ1_0)
    return (double)orc_fp16(tern_scale(type, blk)) * tern_code(type, blk, j);
  if (type == ORC_W_Q4_K) {
    const int sub = j / 32, l = j % 32, p = sub / 2;
    int sc, mn;
    q4k_scale_min(blk, sub, &sc, &mn);
    const uint8_t b = blk[16 + 32 * p + l];
    const int q = (sub & 1) ? (b >> 4) : (b & 0x0f);
    return (double)orc_fp16(rd16(blk)) * sc * q - (double)orc_fp16(rd16(blk + 2)) * mn;
  }
  int q, si;
  q6k_weight(blk, j, &q, &si);
  return (double)orc_fp16(rd16(blk + 208)) * (int8_t)blk[192 + si] * q;
}

int orc_gemv_exact(int type, const float *x, int64_t M, int64_t K, const uint8_t *w,
                   int64_t N, double *y, double *mag) {
  const int B = orc_block_weights(type), BB = orc_block_bytes(type);
  if (!B || K % B) return -1;
  const int64_t row_bytes = K / B * BB;
  double *wr = (double *)malloc(sizeof(double) * (size_t)K);
  if (!wr) return -1;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t k = 0; k < K; ++k) wr[k] = exact_weight(type, w + n * row_bytes, k);
    for (int64_t m = 0; m < M; ++m) {
      double s = 0, a = 0;
      for (int64_t k = 0; k < K; ++k) {
        const double t = (double)x[m * K + k] * wr[k];
        s += t;
        a += fabs(t);
      }
      y[m * N + n] = s;
      if (mag) mag[m * N + n] = a;
    }
  }
  free(wr);
  return 0;
}

/* One invocation's contribution to a row, in the reference's order. */
static float ref_invocation(int type, const float *x, int64_t K, const uint8_t *row, int tid) {
  enum { WG = 64 };
  float acc = 0.0f;
  if (type == ORC_W_F32) {   /* src/kernels.ts:265-275 */
    const float *wf = (const float *)row;
    for (int64_t kv = tid; kv < K / 4; kv += WG) {
      const float *xv = x + 4 * kv, *wv = wf + 4 * kv;
      float dt = xv[0] * wv[0];
      dt = dt + xv[1] * wv[1];
      dt = dt + xv[2] * wv[2];
      dt = dt + xv[3] * wv[3];
      acc = acc + dt;
    }
    return acc;
  }
  if (type == ORC_W_Q4_0 || type == ORC_W_Q4_1) {   /* src/kernels.ts:760-781, :846-867 */
    const int BB = orc_block_bytes(type), qoff = type == ORC_W_Q4_0 ? 2 : 4;
    for (int64_t blk = tid; blk < K / 32; blk += WG) {
      const float *xb = x + 32 * blk;
      const uint8_t *b = row + blk * BB;
      float xs = 0.0f;
      for (int j = 0; j < 32; ++j) xs = xs + xb[j];
      const float d = orc_fp16(rd16(b));
      float qd = 0.0f;
      for (int j = 0; j < 16; ++j) {
        const uint8_t qb = b[qoff + j];
        qd = qd + xb[j] * (float)(qb & 15);
        qd = qd + xb[16 + j] * (float)(qb >> 4);
      }
      if (type == ORC_W_Q4_0) {
        acc = acc + (qd - 8.0f * xs) * d;
      } else {
        const float mn = orc_fp16(rd16(b + 2));
        acc = acc + qd * d;
        acc = acc + xs * mn;
      }
    }
    return acc;
  }
  for (int64_t u = tid; u < K / 32; u += WG) {   /* 32-weight units of the K-quants */
    const int64_t blk = u >> 3;
    const int sub = (int)(u & 7);
    const float *xs_ = x + 32 * u;
    if (type == ORC_W_Q4_K) {   /* src/kernels.ts:943-974 */
      const uint8_t *b = row + blk * 144;
      float xs = 0.0f;
      for (int l = 0; l < 32; ++l) xs = xs + xs_[l];
      const float d = orc_fp16(rd16(b)), dmin = orc_fp16(rd16(b + 2));
      int sc, mn;
      q4k_scale_min(b, sub, &sc, &mn);
      const uint8_t *qb = b + 16 + (sub >> 1) * 32;
      float qd = 0.0f;
      for (int l = 0; l < 32; ++l) {
        const int nib = (sub & 1) ? (qb[l] >> 4) : (qb[l] & 15);
        qd = qd + xs_[l] * (float)nib;
      }
      acc = acc + (d * (float)sc) * qd;
      acc = acc - (dmin * (float)mn) * xs;
    } else {   /* Q6_K, src/kernels.ts:1052-1083 */
      const uint8_t *b = row + blk * 210;
      const int nh = sub >> 2, qg = sub & 3;
      const float d = orc_fp16(rd16(b + 208));
      const uint8_t *ql = b + nh * 64 + (qg & 1) * 32, *qh = b + 128 + nh * 32;
      const float sc0 = (float)(int8_t)b[192 + nh * 8 + qg * 2];
      const float sc1 = (float)(int8_t)b[192 + nh * 8 + qg * 2 + 1];
      float s0 = 0.0f, s1 = 0.0f;
      for (int l = 0; l < 32; ++l) {
        const int lo = qg >= 2 ? (ql[l] >> 4) : (ql[l] & 15);
        const float q = (float)((lo | (((qh[l] >> (2 * qg)) & 3) << 4)) - 32);
        if (l < 16) s0 = s0 + xs_[l] * q;
        else s1 = s1 + xs_[l] * q;
      }
      const float t0 = sc0 * s0, t1 = sc1 * s1;
      acc = acc + d * (t0 + t1);
    }
  }
  return acc;
}

int orc_gemv_ref(int type, const float *x, int64_t M, int64_t K, const uint8_t *w, int64_t N,
                 float *y) {
  const int B = orc_block_weights(type), BB = orc_block_bytes(type);
  if (!B || K % B || (type == ORC_W_F32 && K % 4)) return -1;
  if (type == ORC_W_Q1_0 || type == ORC_W_PQ2_0 || type == ORC_W_PTQ1_0) return -1;
  const int64_t row_bytes = K / B * BB;
  float sdata[64];
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      for (int t = 0; t < 64; ++t) sdata[t] = ref_invocation(type, x + m * K, K, w + n * row_bytes, t);
      for (int s = 32; s > 0; s >>= 1)   /* src/kernels.ts:783-787 */
        for (int t = 0; t < s; ++t) sdata[t] = sdata[t] + sdata[t + s];
      y[m * N + n] = sdata[0];
    }
  }
  return 0;
}

/* src/kernels.ts:177-227 (hadamard_512, mode 0): pre-signs, nine butterfly
 * stages h = 1 .. 256 over pairs (j, j + h), binary32 norm. */
int orc_hadamard512(float *x, int64_t rows, int64_t width, const float *signs) {
  if (width <= 0 || width % 512) return -1;
  const float norm = (float)0.04419417382415922;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c0 = 0; c0 < width; c0 += 512) {
      float *v = x + r * width + c0;
      if (signs)
        for (int i = 0; i < 512; ++i) v[i] = v[i] * signs[c0 + i];
      for (int h = 1; h < 512; h <<= 1)
        for (int i = 0; i < 512; i += 2 * h)
          for (int j = i; j < i + h; ++j) {
            const float a = v[j], b = v[j + h];
            v[j] = a + b;
            v[j + h] = a - b;
          }
      for (int i = 0; i < 512; ++i) v[i] = v[i] * norm;
    }
  }
  return 0;
}
