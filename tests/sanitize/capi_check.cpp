// The C ABI (include/hachiue_sampler.h) with its host code built under
// AddressSanitizer and UndefinedBehaviorSanitizer (the device code is built
// as usual): every entry point once or more, on small inputs, through the
// paths whose host code does the most work (plan building and routing of a
// mixed batch, the host copy-back of penalised entries, split rows, the
// two-pass large-k retry lists, the no-allocation entry point, the planar
// lm_head split, the decode step, timing).  Results are checked loosely here
// (return codes, token ranges); parity is the pytest suites' job.  Without a
// GPU only the host-side argument checks run.  Exit 0: no sanitizer report.
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "hachiue_sampler.h"

namespace {

uint64_t g_rs = 0x9E3779B97F4A7C15ull;
uint64_t rnd() {
  g_rs ^= g_rs << 13;
  g_rs ^= g_rs >> 7;
  g_rs ^= g_rs << 17;
  return g_rs;
}
float unif() { return (float)((rnd() >> 40) * (1.0 / 16777216.0)); }

int g_fail = 0;
#define OK(x)                                                                      \
  do {                                                                             \
    const int rc_ = (x);                                                           \
    if (rc_ != HS_OK) {                                                            \
      fprintf(stderr, "line %d: %s -> %d (%s)\n", __LINE__, #x, rc_, hs_last_error()); \
      ++g_fail;                                                                    \
    }                                                                              \
  } while (0)
#define EXPECT(c)                                                         \
  do {                                                                    \
    if (!(c)) {                                                           \
      fprintf(stderr, "line %d: check failed: %s\n", __LINE__, #c);      \
      ++g_fail;                                                           \
    }                                                                     \
  } while (0)

template <typename T>
T *dev(const std::vector<T> &h) {
  void *p = nullptr;
  if (hipMalloc(&p, sizeof(T) * (h.size() ? h.size() : 1)) != hipSuccess) abort();
  if (!h.empty() && hipMemcpy(p, h.data(), sizeof(T) * h.size(), hipMemcpyHostToDevice) != hipSuccess)
    abort();
  return static_cast<T *>(p);
}

template <typename T>
std::vector<T> host(const T *d, size_t n) {
  std::vector<T> h(n);
  if (hipMemcpy(h.data(), d, sizeof(T) * n, hipMemcpyDeviceToHost) != hipSuccess) abort();
  return h;
}

hs_sample_config cfg(double t, double k, double p, double minp, double rep, double pres,
                     double freq) {
  hs_sample_config c;
  c.temperature = t;
  c.top_k = k;
  c.top_p = p;
  c.min_p = minp;
  c.repetition_penalty = rep;
  c.presence_penalty = pres;
  c.frequency_penalty = freq;
  return c;
}

void host_only_checks() {
  EXPECT(hs_abi_version() == 1);
  hs_sample_config c;
  hs_config_default(&c);
  EXPECT(c.temperature == 0.6 && c.top_k == 20);
  float lg[4] = {1, 2, 3, 4};
  int32_t tok = 0;
  EXPECT(hs_sample_logits(nullptr, lg, 4, nullptr, 0, &c, 0.5, &tok) == HS_ERR_INVALID_ARGUMENT);
  EXPECT(hs_context_destroy(nullptr) == HS_OK);
  EXPECT(hs_context_create(0, nullptr) == HS_ERR_INVALID_ARGUMENT);
  EXPECT(hs_split_blocks(14, nullptr, 1, nullptr, nullptr) == HS_ERR_INVALID_ARGUMENT);
  for (int type : {41, 142, 143}) {
    const int qb = type == 41 ? 16 : type == 142 ? 32 : 26;
    for (int64_t n : {0, 1, 7, 300}) {
      std::vector<uint8_t> blocks((size_t)n * (qb + 2) + 1), q((size_t)n * qb + 1), s((size_t)n * 2 + 1);
      for (auto &b : blocks) b = (uint8_t)rnd();
      OK(hs_split_blocks(type, blocks.data(), n, q.data(), s.data()));
    }
  }
  hs_weights w;
  memset(&w, 0, sizeof w);
  EXPECT(hs_gemv_device_ex(nullptr, nullptr, 1, 1, &w, nullptr, 1, nullptr) ==
         HS_ERR_INVALID_ARGUMENT);
}

void sampling(hs_context *ctx) {
  const int V = 40000, R = 12;
  std::vector<float> logits((size_t)R * V);
  for (auto &v : logits) v = unif() * 8.f - 4.f;
  for (int i = 0; i < V; i += 97) logits[(size_t)3 * V + i] = 9.f;   // a tie group
  std::vector<int32_t> ids;
  std::vector<int64_t> off(1, 0);
  for (int r = 0; r < R; ++r) {
    const int n = r % 4 == 0 ? 0 : (int)(rnd() % 600);
    for (int i = 0; i < n; ++i) ids.push_back(rnd() % 17 == 0 ? -5 : (int32_t)(rnd() % V));
    off.push_back((int64_t)ids.size());
  }
  std::vector<hs_sample_config> cs;
  for (int r = 0; r < R; ++r) {
    switch (r % 6) {
      case 0: cs.push_back(cfg(0.0, 20, 0.95, 0, 1.3, 0, 0)); break;            // greedy
      case 1: cs.push_back(cfg(0.7, 40, 0.9, 0, 1.1, 0, 0)); break;             // row kernel
      case 2: cs.push_back(cfg(1.0, 500, 0.95, 0.02, 1.0, 0.4, 0.2)); break;    // mid + pf
      case 3: cs.push_back(cfg(1.0, INFINITY, 0.98, 0, 1.0, 0, 0)); break;      // k = V
      case 4: cs.push_back(cfg(0.9, 3000, 0.9, 0, 1.2, 0, 0)); break;           // large k
      default: cs.push_back(cfg(NAN, 2.5, NAN, NAN, 1.0, 0, 0)); break;
    }
  }
  std::vector<double> us(R);
  for (auto &u : us) u = unif();
  std::vector<int32_t> tok(R, -7);

  // host buffers: one row, then the batch
  std::vector<float> row(logits.begin(), logits.begin() + V);
  int32_t t1 = -7;
  OK(hs_sample_logits(ctx, row.data(), V, ids.data(), off[1], &cs[1], us[1], &t1));
  EXPECT(t1 >= 0 && t1 < V);
  std::vector<float> lb = logits;
  OK(hs_sample_logits_batch(ctx, lb.data(), R, V, V, ids.data(), off.data(), cs.data(), us.data(),
                            tok.data()));
  for (int r = 0; r < R; ++r) EXPECT(tok[r] >= -1 && tok[r] < V);

  // device buffers: plain, with candidate outputs, without allocation
  float *d_l = dev(logits);
  int32_t *d_ids = dev(ids);
  int64_t *d_off = dev(off);
  double *d_u = dev(us);
  int32_t *d_t = dev(tok);
  OK(hs_sample_batch_device(ctx, d_l, R, V, V, d_ids, d_off, cs.data(), d_u, d_t, nullptr));
  const int cap = 64;
  int32_t *d_cid = dev(std::vector<int32_t>((size_t)R * cap));
  float *d_cp = dev(std::vector<float>((size_t)R * cap));
  int32_t *d_cc = dev(std::vector<int32_t>(R)), *d_cut = dev(std::vector<int32_t>(R));
  uint32_t *d_fl = dev(std::vector<uint32_t>(R));
  OK(hs_sample_batch_device_ex(ctx, d_l, R, V, V, d_ids, d_off, cs.data(), d_u, d_t, cap, d_cid,
                               d_cp, d_cc, d_cut, d_fl, nullptr));
  OK(hs_sample_batch_device_noalloc(ctx, d_l, R, V, V, d_ids, d_off, cs.data(), d_u, d_t, nullptr));
  OK(hs_sample_batch_device_noalloc(ctx, d_l, 5, V, V, d_ids, d_off, cs.data(), d_u, d_t, nullptr));
  (void)hipDeviceSynchronize();
  for (int32_t t : host(d_t, R)) EXPECT(t >= -1 && t < V);

  // a small batch: split rows
  OK(hs_sample_batch_device(ctx, d_l, 2, V, V, d_ids, d_off, cs.data() + 1, d_u, d_t, nullptr));
  // the greedy route
  std::vector<int32_t> am(R);
  OK(hs_argmax(ctx, logits.data(), R, V, V, am.data()));
  OK(hs_argmax_device(ctx, d_l, R, V, V, d_t, nullptr));

  // one decode step with rings
  const int64_t cap_ring = 256;
  std::vector<int32_t> ring((size_t)R * cap_ring, 0);
  std::vector<int64_t> len(R, 3);
  int32_t *d_ring = dev(ring);
  int64_t *d_len = dev(len);
  int32_t *d_done = dev(std::vector<int32_t>(R, 0));
  int32_t *d_stop = dev(std::vector<int32_t>{1, 2, 3});
  OK(hs_decode_step_device(ctx, d_l, R, V, V, d_ring, cap_ring, d_len, d_done, d_stop, 3,
                           cs.data(), d_u, d_t, nullptr));
  (void)hipDeviceSynchronize();
  for (void *p : {(void *)d_l, (void *)d_ids, (void *)d_off, (void *)d_u, (void *)d_t,
                  (void *)d_cid, (void *)d_cp, (void *)d_cc, (void *)d_cut, (void *)d_fl,
                  (void *)d_ring, (void *)d_len, (void *)d_done, (void *)d_stop})
    (void)hipFree(p);
}

void lm_head(hs_context *ctx) {
  const int K = 1024, N = 3001, M = 2;
  std::vector<float> x((size_t)M * K);
  for (auto &v : x) v = unif() - 0.5f;
  float *d_x = dev(x);
  float *d_y = dev(std::vector<float>((size_t)M * N));
  // Q6_K in GGUF blocks
  std::vector<uint8_t> q6((size_t)N * (K / 256) * 210);
  for (auto &b : q6) b = (uint8_t)rnd();
  for (size_t blk = 0; blk < q6.size() / 210; ++blk) {   // finite binary16 scales
    q6[blk * 210 + 208] = 0x00;
    q6[blk * 210 + 209] = 0x20;
  }
  uint8_t *d_q6 = dev(q6);
  OK(hs_gemv_device(ctx, d_x, M, K, K, d_q6, 14, N, d_y, N, nullptr));
  // PTQ1_0 split on the host, folded with the Hadamard rotation
  const int64_t nblk = (int64_t)N * (K / 128);
  std::vector<uint8_t> raw((size_t)nblk * 28), q((size_t)nblk * 26), s((size_t)nblk * 2);
  for (auto &b : raw) b = (uint8_t)rnd();
  for (int64_t b = 0; b < nblk; ++b) {
    raw[(size_t)b * 28 + 26] = 0x00;
    raw[(size_t)b * 28 + 27] = 0x20;
  }
  OK(hs_split_blocks(143, raw.data(), nblk, q.data(), s.data()));
  uint8_t *d_q = dev(q), *d_s = dev(s);
  std::vector<float> sg(K);
  for (auto &v : sg) v = (rnd() & 1) ? 1.f : -1.f;
  float *d_sg = dev(sg);
  hs_weights w;
  w.type = 143;
  w.rows = N;
  w.cols = K;
  w.hadamard = 1;
  w.data = d_q;
  w.scales16 = d_s;
  w.signs = d_sg;
  OK(hs_gemv_device_ex(ctx, d_x, M, K, &w, d_y, N, nullptr));
  std::vector<hs_sample_config> cs(M, cfg(0.8, 40, 0.9, 0, 1.1, 0, 0));
  std::vector<int32_t> ids{1, 2, 3, 4};
  std::vector<int64_t> off{0, 2, 4};
  std::vector<double> us{0.3, 0.7};
  int32_t *d_ids = dev(ids);
  int64_t *d_off = dev(off);
  double *d_u = dev(us);
  int32_t *d_t = dev(std::vector<int32_t>(M));
  OK(hs_lm_head_sample_device_ex(ctx, d_x, M, K, &w, d_y, N, d_ids, d_off, cs.data(), d_u, d_t,
                                 nullptr));
  OK(hs_lm_head_sample_device(ctx, d_x, M, K, K, d_q6, 14, N, d_y, N, d_ids, d_off, cs.data(),
                              d_u, d_t, nullptr));
  (void)hipDeviceSynchronize();
  for (int32_t t : host(d_t, M)) EXPECT(t >= 0 && t < N);
  for (void *p : {(void *)d_x, (void *)d_y, (void *)d_q6, (void *)d_q, (void *)d_s, (void *)d_sg,
                  (void *)d_ids, (void *)d_off, (void *)d_u, (void *)d_t})
    (void)hipFree(p);
}

}  // namespace

int main() {
  host_only_checks();
  hs_context *ctx = nullptr;
  if (hs_context_create(0, &ctx) != HS_OK) {
    printf("no GPU (%s): host-side checks only, %d failed\n", hs_last_error(), g_fail);
    return g_fail ? 1 : 0;
  }
  OK(hs_context_set_timing(ctx, 1));
  sampling(ctx);
  lm_head(ctx);
  double ms[16];
  int64_t calls = 0;
  OK(hs_context_kernel_times(ctx, ms, 16, &calls));
  EXPECT(calls > 0);
  OK(hs_context_set_timing(ctx, 0));
  sampling(ctx);
  OK(hs_context_destroy(ctx));
  if (g_fail) {
    fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  printf("C ABI sanitizer run: ok\n");
  return 0;
}
