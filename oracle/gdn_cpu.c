/*
 * gdn_cpu.c — C/OpenMP fp32 restatement of the gated delta rule.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, and the timed
 * "port" CPU baseline of bench.py.  Never linked into the product.
 *
 * The reference repository contains no gated-delta-rule code; the
 * operator semantics follow transformers
 * models/qwen3_next/modeling_qwen3_next.py (read as text):
 *   gdn_cpu_recurrent_fwd  token loop, :490-501
 *   gdn_cpu_chunk_fwd      chunked UT/WY form, :407-446
 * Inputs are fp32 arrays (the bf16 values of the GPU run, upcast);
 * layouts and argument meanings are those of include/gdn.h.
 * Parallel over (sequence, v-head) pairs with OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define CH 64

static void seq_bounds(const int32_t* cu, int n, int T, int* s, int* e) {
  if (cu) {
    *s = cu[n];
    *e = cu[n + 1];
  } else {
    *s = n * T;
    *e = *s + T;
  }
}

static void l2n(float* x, int K) {
  double ss = 0;
  for (int i = 0; i < K; ++i) ss += (double)x[i] * x[i];
  float inv = (float)(1.0 / sqrt(ss + 1e-6));
  for (int i = 0; i < K; ++i) x[i] *= inv;
}

/* Token recurrence (definition), fp32 or fp64 accumulation of the state. */
int gdn_cpu_recurrent_fwd(const float* q, const float* k, const float* v, const float* g,
                          const float* beta, const float* h0, float* ht, float* o,
                          const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V,
                          int N, float scale, int l2norm, int nthreads) {
  if (Hv % Hqk) return -2;
  const int G = Hv / Hqk;
  (void)B;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (long task = 0; task < (long)N * Hv; ++task) {
    const int n = (int)(task / Hv), h = (int)(task % Hv), hq = h / G;
    float* S = (float*)malloc(sizeof(float) * K * V);
    float* kv = (float*)malloc(sizeof(float) * V);
    float* kt = (float*)malloc(sizeof(float) * K);
    float* qt = (float*)malloc(sizeof(float) * K);
    const size_t tile = ((size_t)n * Hv + h) * K * V;
    if (h0) memcpy(S, h0 + tile, sizeof(float) * K * V);
    else memset(S, 0, sizeof(float) * K * V);
    int s, e;
    seq_bounds(cu, n, T, &s, &e);
    for (int t = s; t < e; ++t) {
      memcpy(kt, k + ((size_t)t * Hqk + hq) * K, sizeof(float) * K);
      memcpy(qt, q + ((size_t)t * Hqk + hq) * K, sizeof(float) * K);
      if (l2norm) { l2n(kt, K); l2n(qt, K); }
      const float eg = expf(g[(size_t)t * Hv + h]);
      const float bt = beta[(size_t)t * Hv + h];
      const float* vt = v + ((size_t)t * Hv + h) * V;
      for (int j = 0; j < V; ++j) kv[j] = 0.f;
      for (int i = 0; i < K * V; ++i) S[i] *= eg;
      for (int i = 0; i < K; ++i)
        for (int j = 0; j < V; ++j) kv[j] += S[i * V + j] * kt[i];
      for (int j = 0; j < V; ++j) kv[j] = bt * (vt[j] - kv[j]);
      for (int i = 0; i < K; ++i)
        for (int j = 0; j < V; ++j) S[i * V + j] += kt[i] * kv[j];
      float* ot = o + ((size_t)t * Hv + h) * V;
      for (int j = 0; j < V; ++j) ot[j] = 0.f;
      for (int i = 0; i < K; ++i)
        for (int j = 0; j < V; ++j) ot[j] += S[i * V + j] * qt[i];
      for (int j = 0; j < V; ++j) ot[j] *= scale;
    }
    if (ht) memcpy(ht + tile, S, sizeof(float) * K * V);
    free(S); free(kv); free(kt); free(qt);
  }
  return 0;
}

/* Chunked form (chunk 64), fp32. */
int gdn_cpu_chunk_fwd(const float* q, const float* k, const float* v, const float* g,
                      const float* beta, const float* h0, float* ht, float* o,
                      const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N,
                      float scale, int l2norm, int nthreads) {
  if (Hv % Hqk || V > 128) return -2;
  const int G = Hv / Hqk;
  (void)B;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (long task = 0; task < (long)N * Hv; ++task) {
    const int n = (int)(task / Hv), h = (int)(task % Hv), hq = h / G;
    float* S = (float*)malloc(sizeof(float) * K * V);
    float* Qc = (float*)malloc(sizeof(float) * CH * K);
    float* Kc = (float*)malloc(sizeof(float) * CH * K);
    float* Vc = (float*)malloc(sizeof(float) * CH * V);
    float* W = (float*)malloc(sizeof(float) * CH * K);
    float* Vn = (float*)malloc(sizeof(float) * CH * V);
    float* A = (float*)malloc(sizeof(float) * CH * CH);
    float* Tm = (float*)malloc(sizeof(float) * CH * CH);
    float* P = (float*)malloc(sizeof(float) * CH * CH);
    float Gc[CH], Bc[CH], eG[CH];
    const size_t tile = ((size_t)n * Hv + h) * K * V;
    if (h0) memcpy(S, h0 + tile, sizeof(float) * K * V);
    else memset(S, 0, sizeof(float) * K * V);
    int s, e;
    seq_bounds(cu, n, T, &s, &e);
    for (int t0 = s; t0 < e; t0 += CH) {
      const int L = (e - t0) < CH ? (e - t0) : CH;
      float run = 0.f;
      for (int i = 0; i < L; ++i) {
        const size_t tq = ((size_t)(t0 + i) * Hqk + hq) * K;
        memcpy(Qc + i * K, q + tq, sizeof(float) * K);
        memcpy(Kc + i * K, k + tq, sizeof(float) * K);
        if (l2norm) { l2n(Qc + i * K, K); l2n(Kc + i * K, K); }
        memcpy(Vc + i * V, v + ((size_t)(t0 + i) * Hv + h) * V, sizeof(float) * V);
        run += g[(size_t)(t0 + i) * Hv + h];
        Gc[i] = run;
        eG[i] = expf(run);
        Bc[i] = beta[(size_t)(t0 + i) * Hv + h];
      }
      /* A = strict_lower(beta_i k_i.k_j Gam_ij), P = lower_incl(q_i.k_j Gam_ij) */
      for (int i = 0; i < L; ++i) {
        for (int j = 0; j <= i; ++j) {
          float kk = 0.f, qk = 0.f;
          for (int d = 0; d < K; ++d) {
            kk += Kc[i * K + d] * Kc[j * K + d];
            qk += Qc[i * K + d] * Kc[j * K + d];
          }
          const float gam = expf(Gc[i] - Gc[j]);
          A[i * CH + j] = (j < i) ? Bc[i] * kk * gam : 0.f;
          P[i * CH + j] = qk * gam;
        }
      }
      /* Tm = (I + A)^-1 by forward substitution (rows) */
      for (int i = 0; i < L; ++i) {
        for (int c = 0; c < L; ++c) Tm[i * CH + c] = (i == c) ? 1.f : 0.f;
        for (int j = 0; j < i; ++j) {
          const float a = A[i * CH + j];
          for (int c = 0; c <= j; ++c) Tm[i * CH + c] -= a * Tm[j * CH + c];
        }
      }
      /* W = Tm diag(beta e^G) K ; Vn = Tm diag(beta) V - W S */
      for (int i = 0; i < L; ++i) {
        float* wi = W + i * K;
        float* vi = Vn + i * V;
        for (int d = 0; d < K; ++d) wi[d] = 0.f;
        for (int c = 0; c < V; ++c) vi[c] = 0.f;
        for (int j = 0; j <= i; ++j) {
          const float tb = Tm[i * CH + j] * Bc[j];
          const float tw = tb * eG[j];
          for (int d = 0; d < K; ++d) wi[d] += tw * Kc[j * K + d];
          for (int c = 0; c < V; ++c) vi[c] += tb * Vc[j * V + c];
        }
        for (int d = 0; d < K; ++d) {
          const float wd = wi[d];
          const float* sd = S + (size_t)d * V;
          for (int c = 0; c < V; ++c) vi[c] -= wd * sd[c];
        }
      }
      /* o = scale (e^G (Q S) + P Vn) */
      for (int i = 0; i < L; ++i) {
        float* oi = o + ((size_t)(t0 + i) * Hv + h) * V;
        float acc[128];
        for (int c = 0; c < V; ++c) acc[c] = 0.f;
        for (int d = 0; d < K; ++d) {
          const float qd = Qc[i * K + d];
          const float* sd = S + (size_t)d * V;
          for (int c = 0; c < V; ++c) acc[c] += qd * sd[c];
        }
        for (int c = 0; c < V; ++c) acc[c] *= eG[i];
        for (int j = 0; j <= i; ++j) {
          const float p = P[i * CH + j];
          for (int c = 0; c < V; ++c) acc[c] += p * Vn[j * V + c];
        }
        for (int c = 0; c < V; ++c) oi[c] = scale * acc[c];
      }
      /* S = e^G_L S + (K * e^(G_L - G))^T Vn */
      const float egl = expf(Gc[L - 1]);
      for (int j = 0; j < L; ++j) {
        const float dj = expf(Gc[L - 1] - Gc[j]);
        for (int c = 0; c < V; ++c) Vn[j * V + c] *= dj;
      }
      for (int d = 0; d < K; ++d) {
        float* sd = S + (size_t)d * V;
        for (int c = 0; c < V; ++c) sd[c] *= egl;
        for (int j = 0; j < L; ++j) {
          const float kd = Kc[j * K + d];
          const float* vj = Vn + j * V;
          for (int c = 0; c < V; ++c) sd[c] += kd * vj[c];
        }
      }
    }
    if (ht) memcpy(ht + tile, S, sizeof(float) * K * V);
    free(S); free(Qc); free(Kc); free(Vc); free(W); free(Vn); free(A); free(Tm); free(P);
  }
  return 0;
}

int gdn_cpu_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
