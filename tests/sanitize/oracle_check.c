/*
 * The CPU oracle (oracle/sampler_oracle.c, oracle/lmhead_oracle.c) under
 * AddressSanitizer and UndefinedBehaviorSanitizer: every entry point on
 * random and adversarial inputs (ties, NaN, +-Infinity, -0, fractional /
 * NaN / infinite topK, k above the finite count, histories with ids out of
 * range and longer than 128, every weight format, the Hadamard rotation).
 * Also checks that the heap scan equals the literal scan.  Exit 0: no
 * sanitizer report and every check held.  Built and run by
 * tests/test_sanitize.py (gcc -fsanitize=address,undefined).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lmhead_oracle.h"
#include "sampler_oracle.h"

static uint64_t rs = 88172645463325252ull;
static uint64_t rnd(void) {
  rs ^= rs << 13;
  rs ^= rs >> 7;
  rs ^= rs << 17;
  return rs;
}
static double unif(void) { return (double)(rnd() >> 11) * (1.0 / 9007199254740992.0); }
static float special(void) {
  switch (rnd() % 8) {
    case 0: return NAN;
    case 1: return INFINITY;
    case 2: return -INFINITY;
    case 3: return -0.0f;
    case 4: return 0.0f;
    default: return (float)((int)(rnd() % 7) - 3);
  }
}

static int fails = 0;
#define CHECK(c)                                                 \
  do {                                                           \
    if (!(c)) {                                                  \
      fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
      ++fails;                                                   \
    }                                                            \
  } while (0)

static void sampler_cases(void) {
  const double topks[] = {40, 1, 2.7, 0, -3, 64, 700, INFINITY, NAN, 1e9};
  const double temps[] = {0.7, 0.0, -1.0, 1.3, NAN, 1e-3};
  for (int it = 0; it < 600; ++it) {
    const int64_t V = 1 + (int64_t)(rnd() % 3000);
    float *a = malloc(sizeof(float) * (size_t)V), *b = malloc(sizeof(float) * (size_t)V);
    const int kind = (int)(rnd() % 4);
    for (int64_t i = 0; i < V; ++i) {
      float v = (float)(unif() * 8 - 4);
      if (kind == 1) v = roundf(v);
      if (kind == 2 && rnd() % 5 == 0) v = special();
      if (kind == 3) v = (rnd() % 3 == 0) ? -INFINITY : roundf(v);
      a[i] = v;
    }
    memcpy(b, a, sizeof(float) * (size_t)V);
    int64_t hl = (int64_t)(rnd() % 400);
    int32_t *h = malloc(sizeof(int32_t) * (size_t)(hl + 1));
    for (int64_t i = 0; i < hl; ++i)
      h[i] = (rnd() % 9 == 0) ? (int32_t)(rnd() % 5) - 2 + (int32_t)(rnd() % 2) * (int32_t)V
                               : (int32_t)(rnd() % (uint64_t)V);
    orc_config c;
    c.temperature = temps[rnd() % 6];
    c.top_k = topks[rnd() % 10];
    c.top_p = (rnd() % 4 == 0) ? NAN : unif();
    c.min_p = (rnd() % 3 == 0) ? unif() : 0.0;
    c.repetition_penalty = (rnd() % 2) ? 1.0 + unif() : 1.0;
    c.presence_penalty = (rnd() % 3 == 0) ? unif() - 0.3 : 0.0;
    c.frequency_penalty = (rnd() % 3 == 0) ? unif() * 0.5 : 0.0;
    const double u = (rnd() % 10 == 0) ? 0.0 : unif();
    const int64_t cap = 64;
    int32_t ia[64], ib[64];
    float va[64], vb[64], pa[64], pb[64];
    orc_result ra, rb;
    CHECK(orc_sample_row(a, V, h, hl, &c, u, ORC_TOPK_LITERAL, &ra, ia, va, pa, cap) == 0);
    CHECK(orc_sample_row(b, V, h, hl, &c, u, ORC_TOPK_HEAP, &rb, ib, vb, pb, cap) == 0);
    CHECK(ra.token == rb.token && ra.n == rb.n && ra.cutoff == rb.cutoff);
    CHECK(memcmp(a, b, sizeof(float) * (size_t)V) == 0);
    const int64_t m = ra.n < cap ? ra.n : cap;
    CHECK(m <= 0 || memcmp(ia, ib, sizeof(int32_t) * (size_t)m) == 0);
    int32_t t1 = 0, t2 = 0;
    orc_wgsl_argmax(a, 1, V, V, &t1);
    orc_wasm_greedy(a, 1, V, V, &t2);
    CHECK(t1 >= 0 && t1 < V && t2 >= 0 && t2 < V);
    const int64_t k = orc_resolve_k(c.top_k, V);
    int32_t *sid = malloc(sizeof(int32_t) * (size_t)k);
    float *sv = malloc(sizeof(float) * (size_t)k);
    CHECK(orc_topk_slots(a, V, k, ORC_TOPK_HEAP, sid, sv) == 0);
    free(sid);
    free(sv);
    free(a);
    free(b);
    free(h);
  }
  /* a batch with strides */
  const int64_t R = 5, V = 777, S = 800;
  float *lg = malloc(sizeof(float) * (size_t)(R * S));
  for (int64_t i = 0; i < R * S; ++i) lg[i] = (float)(unif() * 6 - 3);
  int32_t ids[10] = {1, 2, 3, 776, 777, -1, 5, 5, 5, 9};
  int64_t off[6] = {0, 2, 2, 5, 8, 10};
  orc_config cf[5];
  double us[5];
  for (int r = 0; r < 5; ++r) {
    cf[r] = (orc_config){0.8, 40, 0.9, 0, 1.2, 0.1 * r, 0.05, };
    us[r] = unif();
  }
  orc_result res[5];
  CHECK(orc_sample_batch(lg, R, S, V, ids, off, cf, us, ORC_TOPK_HEAP, res, NULL, NULL, NULL, 0) == 0);
  free(lg);
}

static void lmhead_cases(void) {
  const int types[] = {ORC_W_F32, ORC_W_Q4_0, ORC_W_Q4_1, ORC_W_Q4_K, ORC_W_Q6_K,
                       ORC_W_Q1_0, ORC_W_PQ2_0, ORC_W_PTQ1_0};
  for (int t = 0; t < 8; ++t) {
    const int type = types[t];
    const int B = orc_block_weights(type), BB = orc_block_bytes(type);
    const int64_t K = 512, N = 7, M = 2;
    const int64_t rb = K / B * BB;
    uint8_t *w = malloc((size_t)(N * rb));
    for (int64_t i = 0; i < N * rb; ++i) w[i] = (uint8_t)rnd();
    if (type == ORC_W_F32)
      for (int64_t i = 0; i < N * K; ++i) ((float *)w)[i] = (float)(unif() - 0.5);
    float *x = malloc(sizeof(float) * (size_t)(M * K));
    for (int64_t i = 0; i < M * K; ++i) x[i] = (float)(unif() * 2 - 1);
    float *row = malloc(sizeof(float) * (size_t)K);
    CHECK(orc_dequant_row(type, w, K, row) == 0);
    double *y = malloc(sizeof(double) * (size_t)(M * N)), *mag = malloc(sizeof(double) * (size_t)(M * N));
    CHECK(orc_gemv_exact(type, x, M, K, w, N, y, mag) == 0);
    float *yr = malloc(sizeof(float) * (size_t)(M * N));
    const int ref = orc_gemv_ref(type, x, M, K, w, N, yr);
    CHECK(ref == 0 || type == ORC_W_Q1_0 || type == ORC_W_PQ2_0 || type == ORC_W_PTQ1_0);
    free(w);
    free(x);
    free(row);
    free(y);
    free(mag);
    free(yr);
  }
  for (int i = 0; i < 65536; ++i) (void)orc_fp16((uint16_t)i);
  float *v = malloc(sizeof(float) * 2048), *s = malloc(sizeof(float) * 1024);
  for (int i = 0; i < 2048; ++i) v[i] = (float)(unif() - 0.5);
  for (int i = 0; i < 1024; ++i) s[i] = (rnd() & 1) ? 1.0f : -1.0f;
  CHECK(orc_hadamard512(v, 2, 1024, s) == 0);
  CHECK(orc_hadamard512(v, 1, 100, NULL) == -1);
  free(v);
  free(s);
}

int main(void) {
  sampler_cases();
  lmhead_cases();
  if (fails) {
    fprintf(stderr, "%d checks failed\n", fails);
    return 1;
  }
  printf("oracle sanitizer run: ok\n");
  return 0;
}
