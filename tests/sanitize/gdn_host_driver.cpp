// Host-side driver for the sanitizer tier (tests/test_sanitize.py).
//
// Linked against an AddressSanitizer + UBSan build of the C ABI (host code
// of avelang_amd/csrc/*.hip; the device code is never launched) and of the
// C oracle (oracle/gdn_cpu.c).  It exercises everything that
// runs on the host without a GPU:
//   - every entry point with invalid arguments: the documented negative
//     code, a non-empty message, and no launch;
//   - every entry point on an empty problem: 0 and no launch;
//   - the cu_seqlens contract check on exact-size heap arrays (an
//     over-read is an ASan error);
//   - the workspace-size functions over a range of shapes;
//   - the C oracle's chunked form against its token recurrence on small
//     random problems in exact-size heap buffers.
// Prints "OK" and exits 0 when every check holds.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../../include/gdn.h"
#include "../../include/gdn_layer.h"

extern "C" {
int gdn_cpu_recurrent_fwd(const float* q, const float* k, const float* v, const float* g,
                          const float* beta, const float* h0, float* ht, float* o,
                          const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V,
                          int N, float scale, int l2norm, int nthreads);
int gdn_cpu_chunk_fwd(const float* q, const float* k, const float* v, const float* g,
                      const float* beta, const float* h0, float* ht, float* o,
                      const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N,
                      float scale, int l2norm, int nthreads);
}

static int failures = 0;

#define EXPECT(cond, what)                                      \
  do {                                                          \
    if (!(cond)) {                                              \
      std::fprintf(stderr, "FAIL %s:%d %s\n", __FILE__, __LINE__, what); \
      ++failures;                                               \
    }                                                           \
  } while (0)

// Distinct fake device addresses: never dereferenced, since every call
// below fails validation or is an empty problem.
static void* fake(int i) { return reinterpret_cast<void*>((uintptr_t)(i + 1) << 28); }
static float* fakef(int i) { return static_cast<float*>(fake(i)); }

static void expect_code(int rc, int code, const char* what) {
  EXPECT(rc == code, what);
  if (rc != 0) EXPECT(std::strlen(gdn_last_error()) > 0, what);
}

static void argument_errors() {
  const void *q = fake(0), *k = fake(1), *v = fake(2);
  float *g = fakef(3), *beta = fakef(4), *ht = fakef(5);
  void* o = fake(6);
  // gdn_chunk_fwd / _fwd_save
  expect_code(gdn_chunk_fwd(nullptr, k, v, g, beta, nullptr, nullptr, o, nullptr, 1, 64, 2, 4,
                            128, 128, 1, 0.1f, 0, fake(9), 1 << 30, nullptr),
              GDN_ERR_NULL, "chunk_fwd null q");
  expect_code(gdn_chunk_fwd(q, k, v, g, beta, nullptr, nullptr, o, nullptr, 1, 64, 2, 4, 96,
                            128, 1, 0.1f, 0, fake(9), 1 << 30, nullptr),
              GDN_ERR_SHAPE, "chunk_fwd K=96");
  expect_code(gdn_chunk_fwd(q, k, v, g, beta, nullptr, nullptr, o, nullptr, 1, 64, 3, 4, 128,
                            128, 1, 0.1f, 0, fake(9), 1 << 30, nullptr),
              GDN_ERR_SHAPE, "chunk_fwd Hv % Hqk");
  expect_code(gdn_chunk_fwd(q, k, v, g, beta, nullptr, nullptr, o,
                            static_cast<const int32_t*>(fake(8)), 2, 64, 2, 4, 128, 128, 2, 0.1f,
                            0, fake(9), 1 << 30, nullptr),
              GDN_ERR_SEQLENS, "chunk_fwd cu_seqlens with B != 1");
  expect_code(gdn_chunk_fwd(q, k, v, g, beta, nullptr, nullptr, o, nullptr, 1, 64, 2, 4, 128,
                            128, 1, 0.1f, 0, nullptr, 0, nullptr),
              GDN_ERR_WORKSPACE, "chunk_fwd no workspace");
  expect_code(gdn_chunk_fwd_save(q, k, v, g, beta, nullptr, nullptr, o, nullptr, 1, 64, 2, 4,
                                 128, 128, 1, 0.1f, 0, fake(9), 16, nullptr),
              GDN_ERR_WORKSPACE, "chunk_fwd_save small workspace");
  expect_code(gdn_chunk_fwd(q, k, v, g, beta, ht, static_cast<float*>(static_cast<void*>(
                                static_cast<char*>(static_cast<void*>(ht)) + 64)),
                            o, nullptr, 1, 64, 2, 4, 128, 128, 1, 0.1f, 0, fake(9), 1 << 30,
                            nullptr),
              GDN_ERR_ALIAS, "chunk_fwd ht overlapping h0");
  // gdn_chunk_bwd
  expect_code(gdn_chunk_bwd(q, k, v, g, beta, nullptr, fake(10), nullptr, nullptr, fake(12),
                            fake(13), fakef(14), fakef(15), nullptr, nullptr, 1, 64, 2, 4, 128,
                            128, 1, 0.1f, 0, 0, fake(9), 1 << 30, nullptr),
              GDN_ERR_NULL, "chunk_bwd null dq");
  expect_code(gdn_chunk_bwd(q, k, v, g, beta, nullptr, fake(10), nullptr, fake(11), fake(11),
                            fake(13), fakef(14), fakef(15), nullptr, nullptr, 1, 64, 2, 4, 128,
                            128, 1, 0.1f, 0, 0, fake(9), 1 << 30, nullptr),
              GDN_ERR_ALIAS, "chunk_bwd dq == dk");
  // recurrent entry points
  expect_code(gdn_recurrent_fwd(q, k, v, g, nullptr, nullptr, nullptr, o, nullptr, 1, 4, 2, 4,
                                128, 128, 1, 0.1f, 0, nullptr),
              GDN_ERR_NULL, "recurrent_fwd null beta");
  expect_code(gdn_recurrent_fwd_indexed(q, k, v, g, beta, fakef(7), fakef(7), o, nullptr, nullptr,
                                        1, 4, 2, 4, 128, 128, 1, 8, 0.1f, 0, nullptr),
              GDN_ERR_NULL, "recurrent_fwd_indexed null indices");
  expect_code(gdn_recurrent_fwd_spec(q, k, v, g, beta, fakef(7), o, nullptr,
                                     static_cast<const int32_t*>(fake(8)), 0, nullptr, 1, 4, 2, 4,
                                     128, 128, 1, 8, 0.1f, 0, nullptr),
              GDN_ERR_SHAPE, "recurrent_fwd_spec index_stride 0");
  expect_code(gdn_recurrent_fwd_spec(q, k, v, g, beta, fakef(7), o, nullptr,
                                     static_cast<const int32_t*>(fake(8)), 2, nullptr, 1, 4, 2, 4,
                                     128, 128, 1, 8, 0.1f, 0, nullptr),
              GDN_ERR_SHAPE, "recurrent_fwd_spec T > index_stride");
  // layer operators
  expect_code(gdn_gating_fwd(nullptr, fake(1), fake(2), fake(3), g, beta, 16, 4, 0, 0, 0, 1.f,
                             20.f, nullptr),
              GDN_ERR_NULL, "gating null A_log");
  expect_code(gdn_l2norm_fwd(fake(1), nullptr, 16, 128, 1e-6f, 0, nullptr), GDN_ERR_NULL,
              "l2norm null y");
  expect_code(gdn_rmsnorm_gated_fwd(fake(1), fake(2), nullptr, fake(4), 16, 128, 1e-6f, 0, 0,
                                    nullptr),
              GDN_ERR_NULL, "rmsnorm null weight");
  expect_code(gdn_causal_conv1d_fwd(nullptr, fake(1), nullptr, nullptr, nullptr, nullptr, fake(2),
                                    1, 64, 16, 4, 1024, 1, 64, 1024, 1, 64, 1, 0, 0, nullptr),
              GDN_ERR_NULL, "conv1d null x");
  expect_code(gdn_causal_conv1d_update(fake(1), nullptr, fake(2), nullptr, nullptr, fake(3), 2,
                                       64, 1, 4, 3, 2, 64, 1, 64, 64, 1, 64, 1, 0, 0, nullptr),
              GDN_ERR_NULL, "conv1d_update null state");
  expect_code(gdn_causal_conv1d_update(fake(1), fake(4), fake(2), nullptr, nullptr, fake(3), 2,
                                       64, 1, 4, 3, 1, 64, 1, 64, 64, 1, 64, 1, 0, 0, nullptr),
              GDN_ERR_SHAPE, "conv1d_update fewer slots than rows");
}

static void empty_problems() {
  const void *q = fake(0), *k = fake(1), *v = fake(2);
  float *g = fakef(3), *beta = fakef(4);
  EXPECT(gdn_chunk_fwd(q, k, v, g, beta, nullptr, nullptr, fake(6), nullptr, 0, 64, 2, 4, 128,
                       128, 0, 0.1f, 0, nullptr, 0, nullptr) == 0, "chunk_fwd B=N=0");
  expect_code(gdn_chunk_fwd(q, k, v, g, beta, nullptr, nullptr, fake(6), nullptr, 1, 64, 2, 4,
                            128, 128, 0, 0.1f, 0, nullptr, 0, nullptr),
              GDN_ERR_SEQLENS, "chunk_fwd N != B without cu_seqlens");
  EXPECT(gdn_recurrent_fwd(q, k, v, g, beta, nullptr, nullptr, fake(6), nullptr, 0, 4, 2, 4, 128,
                           128, 0, 0.1f, 0, nullptr) == 0, "recurrent_fwd B=0");
  EXPECT(gdn_gating_fwd(fake(1), fake(2), fake(3), fake(4), g, beta, 0, 4, 0, 0, 0, 1.f, 20.f,
                        nullptr) == 0, "gating rows=0");
  EXPECT(gdn_l2norm_fwd(fake(1), fake(2), 0, 128, 1e-6f, 0, nullptr) == 0, "l2norm rows=0");
}

static void cu_contract() {
  std::mt19937 rng(7);
  for (int trial = 0; trial < 200; ++trial) {
    const int N = trial % 50;
    // exact-size heap array: reading past cu[N] is an ASan error
    std::vector<int32_t>* cu = new std::vector<int32_t>(N + 1);
    int run = 0;
    for (int n = 0; n <= N; ++n) {
      (*cu)[n] = run;
      run += rng() % 200;
    }
    const int total = (*cu)[N];
    EXPECT(gdn_cu_seqlens_check(cu->data(), N, total) == GDN_OK, "valid cu_seqlens");
    if (N > 0) {
      std::vector<int32_t> bad = *cu;
      bad[1 + rng() % N] = -1;   // a decrease (or a negative start of the next)
      EXPECT(gdn_cu_seqlens_check(bad.data(), N, total) == GDN_ERR_SEQLENS, "decrease found");
      EXPECT(gdn_cu_seqlens_check(cu->data(), N, total + 1) == GDN_ERR_SEQLENS, "total found");
    }
    delete cu;
  }
}

static void workspace_sizes() {
  for (int K : {64, 128})
    for (int T : {0, 1, 63, 64, 65, 8192})
      for (int cu = 0; cu < 2; ++cu)
        for (int l2 = 0; l2 < 2; ++l2) {
          const size_t a = gdn_chunk_workspace_bytes(1, T, 2, 4, K, 128, cu ? 3 : 1, cu, l2);
          const size_t b = gdn_chunk_bwd_workspace_bytes(1, T, 2, 4, K, 128, cu ? 3 : 1, cu, l2);
          EXPECT(b >= a, "backward workspace covers the forward's");
        }
  EXPECT(gdn_chunk_workspace_bytes(-1, 4, 2, 4, 128, 128, 1, 0, 0) == 0, "negative B");
}

static void thread_local_errors() {
  std::string other;
  gdn_cu_seqlens_check(nullptr, 1, 4);   // this thread: a NULL error
  std::thread t([&] {
    const int32_t cu[2] = {1, 4};
    gdn_cu_seqlens_check(cu, 1, 4);
    other = gdn_last_error();
  });
  t.join();
  EXPECT(std::string(gdn_last_error()).find("NULL") != std::string::npos, "own message kept");
  EXPECT(other.find("cu_seqlens[0]") != std::string::npos, "other thread's message");
}

static void oracle_forms_agree() {
  std::mt19937 rng(11);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (int trial = 0; trial < 4; ++trial) {
    const int T = 150 + 37 * trial, Hqk = 2, Hv = 4, K = trial % 2 ? 64 : 128, V = 64;
    const int32_t cuv[4] = {0, 0, 70, T};   // one empty sequence
    const int N = 3;
    std::vector<float> q((size_t)T * Hqk * K), k(q.size()), v((size_t)T * Hv * V),
        g((size_t)T * Hv), beta(g.size()), h0((size_t)N * Hv * K * V);
    for (auto& x : q) x = nd(rng) * 0.3f;
    for (auto& x : k) x = nd(rng) * 0.3f;
    for (auto& x : v) x = nd(rng);
    for (auto& x : g) x = -0.1f * std::fabs(nd(rng));
    for (auto& x : beta) x = 1.f / (1.f + std::exp(-nd(rng)));
    for (auto& x : h0) x = nd(rng) * 0.01f;
    std::vector<float> o1(v.size()), o2(v.size()), s1(h0.size()), s2(h0.size());
    const float scale = 1.f / std::sqrt((float)K);
    EXPECT(gdn_cpu_recurrent_fwd(q.data(), k.data(), v.data(), g.data(), beta.data(), h0.data(),
                                 s1.data(), o1.data(), cuv, 1, T, Hqk, Hv, K, V, N, scale,
                                 trial >= 2, 1) == 0, "recurrent oracle");
    EXPECT(gdn_cpu_chunk_fwd(q.data(), k.data(), v.data(), g.data(), beta.data(), h0.data(),
                             s2.data(), o2.data(), cuv, 1, T, Hqk, Hv, K, V, N, scale, trial >= 2,
                             1) == 0, "chunk oracle");
    double num = 0, den = 0, snum = 0, sden = 0;
    for (size_t i = 0; i < o1.size(); ++i) {
      num += (double)(o1[i] - o2[i]) * (o1[i] - o2[i]);
      den += (double)o1[i] * o1[i];
    }
    for (size_t i = 0; i < s1.size(); ++i) {
      snum += (double)(s1[i] - s2[i]) * (s1[i] - s2[i]);
      sden += (double)s1[i] * s1[i];
    }
    EXPECT(std::sqrt(num / den) < 1e-4, "chunked oracle output matches the recurrence");
    EXPECT(std::sqrt(snum / sden) < 1e-4, "chunked oracle state matches the recurrence");
  }
}

int main() {
  argument_errors();
  empty_problems();
  cu_contract();
  workspace_sizes();
  thread_local_errors();
  oracle_forms_agree();
  if (failures) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("OK\n");
  return 0;
}
