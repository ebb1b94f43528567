// Producer / consumer operators around the gated-delta-net core of a
// Qwen3-Next linear-attention layer, for gfx950: gating (g, beta), row L2
// normalisation, the causal depthwise convolution (prefill and in-place
// decode update) and the gated RMSNorm on the core output.
//
// Semantics follow transformers' Qwen3-Next layer text (models/qwen3_next/
// modeling_qwen3_next.py, 5.15.0): causal_conv1d_update :326-343,
// causal_conv1d_fn :346-365, l2norm :368-371, gating :650-652, gated RMSNorm
// :58-74 applied at :693.  The reference repository has no counterpart;
// its launcher convention (raw pointers + scalars + caller stream,
// python/avelang/backends/amdgpu/driver.py:324-343) is kept.
//
// All of these are HBM-bound elementwise / stencil operators: the kernels
// move 16 bytes per lane per access on their contiguous axis (a wavefront
// covers 1 KiB), keep sliding windows in registers, and compute in fp32.
#include "gdn_common.h"
#include "../../include/gdn_layer.h"

namespace gdn {

// 16-byte vector load / store of VEC consecutive elements (element index
// aligned to VEC).
template <int DT>
__device__ __forceinline__ void ldv(const void* p, long long i, float (&v)[Elt<DT>::VEC]) {
  using E = Elt<DT>;
  const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const typename E::T*>(p) + i);
  const typename E::T* e = reinterpret_cast<const typename E::T*>(&raw);
#pragma unroll
  for (int c = 0; c < E::VEC; ++c) v[c] = E::to_f(e[c]);
}
template <int DT>
__device__ __forceinline__ void stv(void* p, long long i, const float (&v)[Elt<DT>::VEC]) {
  using E = Elt<DT>;
  uint4 raw;
  typename E::T* e = reinterpret_cast<typename E::T*>(&raw);
#pragma unroll
  for (int c = 0; c < E::VEC; ++c) e[c] = E::from_f(v[c]);
  *reinterpret_cast<uint4*>(static_cast<typename E::T*>(p) + i) = raw;
}

// x * sigmoid(x) with the hardware exp and a fast divide (~2 ulp in fp32)
__device__ __forceinline__ float silu_f(float x) { return __fdividef(x, 1.f + __expf(-x)); }

// M consecutive parameters starting at element e0, converted to fp32: 16-byte
// loads when M fills whole vectors of the parameter type (e0 aligned to
// them), element loads otherwise.
template <int M, int WDT>
__device__ __forceinline__ void ld_params_t(const void* p, long long e0, float (&out)[M]) {
  constexpr int PER = Elt<WDT>::VEC;
  if constexpr (M % PER == 0) {
#pragma unroll
    for (int v = 0; v < M / PER; ++v) {
      float tmp[PER];
      ldv<WDT>(p, e0 + v * PER, tmp);
#pragma unroll
      for (int k = 0; k < PER; ++k) out[v * PER + k] = tmp[k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < M; ++k) out[k] = lde<WDT>(p, e0 + k);
  }
}
template <int M>
__device__ __forceinline__ void ld_params(const void* p, long long e0, int wdt, float (&out)[M]) {
  if (wdt == GDN_DTYPE_F32) ld_params_t<M, GDN_DTYPE_F32>(p, e0, out);
  else if (wdt == GDN_DTYPE_BF16) ld_params_t<M, GDN_DTYPE_BF16>(p, e0, out);
  else ld_params_t<M, GDN_DTYPE_F16>(p, e0, out);
}

// -------------------------------------------------------------- gating ----
// g = -exp(A_log[h]) * softplus(a + dt_bias[h]), beta = sigmoid(b); fp32 math
// with the accurate exp / log1p (the decay is exponentiated again downstream).
__global__ __launch_bounds__(256) void gating_kernel(GateIn p, float* g, float* beta, long long n,
                                                     int H) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float gi, bi;
    gate_at(p, i, (int)(i % H), gi, bi);
    g[i] = gi;
    if (beta) beta[i] = bi;
  }
}

// ---------------------------------------------------- gating backward ----
// Gradients of the gating (autograd of TF:650-652) from dg, dbeta:
//   da = dg * -exp(A_log[h]) * softplus'(a + dt_bias[h]),  softplus'(x) =
//        sigmoid(spb x), or 1 where spb x > spt (torch's softplus backward);
//   db = dbeta * beta (1 - beta)  (formed as e^-|b| / (1 + e^-|b|)^2);
//   ddt_bias[h] = sum over rows of da (fp32, before da is rounded to a's type),
//   dA_log[h]   = sum over rows of dg * g   (d(-exp(A)) / dA = -exp(A)).
// Deterministic sums: block blk takes rows [blk R, blk R + R); thread j of
// head h (tph = 256 / H threads per head, consecutive threads consecutive
// heads, so a row's elements are one coalesced access) sums rows j, j + tph,
// .. in order, then the tph partials are summed in order and stored per
// block; gating_bwd_reduce_kernel sums the block partials in order.
__device__ __forceinline__ void st_dt(void* p, long long i, int dt, float v) {
  if (dt == GDN_DTYPE_F32) static_cast<float*>(p)[i] = v;
  else if (dt == GDN_DTYPE_BF16) ste<GDN_DTYPE_BF16>(p, i, v);
  else ste<GDN_DTYPE_F16>(p, i, v);
}
__global__ __launch_bounds__(256) void gating_bwd_kernel(GateIn p, const float* __restrict__ dg,
                                                         const float* __restrict__ dbeta, void* da,
                                                         void* db, float* __restrict__ part,
                                                         long long rows, int H, int R) {
  __shared__ float red[2][256];
  const int tph = 256 / H;
  const int t = threadIdx.x, h = t % H, j = t / H;
  const long long r0 = (long long)blockIdx.x * R;
  const long long r1 = min(rows, r0 + R);
  float sdt = 0.f, sA = 0.f;
  if (j < tph) {
    float neg_a, dtb;
    gate_head(p, h, neg_a, dtb);
    for (long long r = r0 + j; r < r1; r += tph) {
      const long long i = r * H + h;
      const float av = ldp(p.a, i, p.adt);
      float g, unused;
      gate_math(p, neg_a, dtb, av, 0.f, g, unused);
      const float bx = p.spb * (av + dtb);
      const float ex = expf(fminf(bx, p.spt));
      const float dsp = bx > p.spt ? 1.f : ex / (1.f + ex);
      const float dgi = dg[i];
      const float dai = dgi * neg_a * dsp;
      st_dt(da, i, p.adt, dai);
      sdt += dai;
      sA += dgi * g;
      if (db) {
        // beta (1 - beta) = e^-|b| / (1 + e^-|b|)^2, without the cancellation
        // of 1 - beta where beta is near 1
        const float eb = expf(-fabsf(ldp(p.b, i, p.bdt)));
        st_dt(db, i, p.bdt, dbeta[i] * (eb / ((1.f + eb) * (1.f + eb))));
      }
    }
  }
  red[0][t] = sdt;
  red[1][t] = sA;
  __syncthreads();
  if (t < H) {
    float s0 = 0.f, s1 = 0.f;
    for (int jj = 0; jj < tph; ++jj) {
      s0 += red[0][jj * H + t];
      s1 += red[1][jj * H + t];
    }
    part[((size_t)blockIdx.x * H + t) * 2] = s0;
    part[((size_t)blockIdx.x * H + t) * 2 + 1] = s1;
  }
}
__global__ __launch_bounds__(256) void gating_bwd_reduce_kernel(const float* __restrict__ part,
                                                                int nblk, int H, void* dA_log,
                                                                void* ddt, int pdt) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= H) return;
  float s0 = 0.f, s1 = 0.f;
  for (int b = 0; b < nblk; ++b) {
    s0 += part[((size_t)b * H + h) * 2];
    s1 += part[((size_t)b * H + h) * 2 + 1];
  }
  if (ddt) st_dt(ddt, h, pdt, s0);
  if (dA_log) st_dt(dA_log, h, pdt, s1);
}

// Row kernels (l2norm, gated norm): a row of D elements is held by D / VEC
// lanes with one 16-byte access each (LPR lanes per row, 64 / LPR rows per
// wavefront), the row sum is a xor-shuffle over those lanes.
template <int D, int DT>
struct RowShape {
  static constexpr int VEC = Elt<DT>::VEC;
  static constexpr int LPR = D / VEC;          // lanes per row (8 .. 64)
  static constexpr int RPW = 64 / LPR;         // rows per wavefront
  static constexpr int RPB = 4 * RPW;          // rows per 256-lane block
  static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "row shape");
};

template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// -------------------------------------------------------------- l2norm ----
template <int D, int DT>
__global__ __launch_bounds__(256) void l2norm_kernel(const void* x, void* y, long long rows,
                                                     float eps) {
  using RS = RowShape<D, DT>;
  constexpr int N = RS::VEC;
  const long long row = (long long)blockIdx.x * RS::RPB + threadIdx.x / RS::LPR;
  const int part = threadIdx.x % RS::LPR;
  const bool live = row < rows;
  const long long base = (live ? row : 0) * D + part * N;
  float v[N];
  ldv<DT>(x, base, v);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < N; ++c) ss += v[c] * v[c];
  const float r = rsqrtf(group_sum<RS::LPR>(ss) + eps);
#pragma unroll
  for (int c = 0; c < N; ++c) v[c] *= r;
  if (live) stv<DT>(y, base, v);
}

// ---------------------------------------------------------- gated norm ----
// n = round(x * rsqrt(mean x^2 + eps)); out = round(weight * n [rounded when
// the weight has the input's type] * silu(z)).
template <int D, int DT>
__global__ __launch_bounds__(256) void rmsnorm_gated_kernel(const void* x, const void* z,
                                                            const void* weight, void* out,
                                                            long long rows, float eps, int wdt) {
  using RS = RowShape<D, DT>;
  constexpr int N = RS::VEC;
  const long long row = (long long)blockIdx.x * RS::RPB + threadIdx.x / RS::LPR;
  const int part = threadIdx.x % RS::LPR;
  const bool live = row < rows;
  const long long base = (live ? row : 0) * D + part * N;
  float v[N], zv[N];
  ldv<DT>(x, base, v);
  ldv<DT>(z, base, zv);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < N; ++c) ss += v[c] * v[c];
  const float r = rsqrtf(group_sum<RS::LPR>(ss) / D + eps);
  const bool round_w = wdt == DT;
  float wv[N];
  ld_params<N>(weight, part * N, wdt, wv);
#pragma unroll
  for (int c = 0; c < N; ++c) {
    const float nv = round_to<DT>(v[c] * r);
    float wn = wv[c] * nv;
    if (round_w) wn = round_to<DT>(wn);
    v[c] = wn * silu_f(zv[c]);
  }
  if (live) stv<DT>(out, base, v);
}

// ------------------------------------------------------- causal conv1d ----
struct ConvArgs {
  const void* x;
  const void* weight;
  const void* bias;
  const int32_t* seq_idx;
  const void* init;
  void* final_states;
  void* out;
  int B, D, T;
  long long x_sb, x_sd, x_st, o_sb, o_sd, o_st;
  int silu, wdt;
};

// Channel-last layout (x_sd == o_sd == 1): lane = VEC consecutive channels,
// a workgroup = 256 * VEC channels of one time step (one 4 KiB access at
// bf16), each lane walks TT time steps with the last W-1 inputs in
// registers.  Workgroups of one time tile are adjacent in dispatch order, so
// a time step's row is read as a few wide pieces at once (measured: 4.2 TB/s
// against 3.9 with 1 KiB pieces from 4 time tiles per workgroup).
template <int DT, int W>
__global__ __launch_bounds__(256) void conv1d_cl_kernel(ConvArgs a, int TT) {
  constexpr int N = Elt<DT>::VEC;
  constexpr int U = 8;   // time steps whose loads are issued together
  const int d0 = (blockIdx.x * 256 + threadIdx.x) * N;
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * TT;
  if (d0 >= a.D || t0 >= a.T) return;
  const int t1 = min(t0 + TT, a.T);

  float wf[N * W], bs[N];
  ld_params<N * W>(a.weight, (long long)d0 * W, a.wdt, wf);
  if (a.bias) {
    ld_params<N>(a.bias, d0, a.wdt, bs);
  } else {
#pragma unroll
    for (int c = 0; c < N; ++c) bs[c] = 0.f;
  }
  const long long xb = (long long)b * a.x_sb + d0;
  const long long ob = (long long)b * a.o_sb + d0;
  const int32_t* sq = a.seq_idx ? a.seq_idx + (long long)b * a.T : nullptr;

  // window slot j holds the input at t - (W-1) + j (oldest first) and its
  // sequence id (padding before the row start never matches a token)
  float win[W - 1][N];
  int sw[W - 1];
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const int p = t0 - (W - 1) + j;
    if (p >= 0) {
      ldv<DT>(a.x, xb + p * a.x_st, win[j]);
      sw[j] = sq ? sq[p] : 0;
    } else {
#pragma unroll
      for (int c = 0; c < N; ++c)
        win[j][c] = a.init ? lde<DT>(a.init, ((long long)b * a.D + d0 + c) * (W - 1) + (W - 1) + p)
                           : 0.f;
      sw[j] = sq ? -2147483647 - 1 : 0;
    }
  }
  for (int tb = t0; tb < t1; tb += U) {
    float cur[U][N];
    int sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = min(tb + u, t1 - 1);   // clamped: steps past t1 are not used
      ldv<DT>(a.x, xb + t * a.x_st, cur[u]);
      sc[u] = sq ? sq[t] : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tb + u >= t1) break;
      float acc[N];
#pragma unroll
      for (int c = 0; c < N; ++c) acc[c] = bs[c] + wf[c * W + W - 1] * cur[u][c];
#pragma unroll
      for (int j = 0; j < W - 1; ++j) {
        if (sw[j] == sc[u]) {
#pragma unroll
          for (int c = 0; c < N; ++c) acc[c] += wf[c * W + j] * win[j][c];
        }
      }
      if (a.silu) {
#pragma unroll
        for (int c = 0; c < N; ++c) acc[c] = silu_f(acc[c]);
      }
      stv<DT>(a.out, ob + (tb + u) * a.o_st, acc);
#pragma unroll
      for (int j = 0; j + 1 < W - 1; ++j) {
#pragma unroll
        for (int c = 0; c < N; ++c) win[j][c] = win[j + 1][c];
        sw[j] = sw[j + 1];
      }
#pragma unroll
      for (int c = 0; c < N; ++c) win[W - 2][c] = cur[u][c];
      sw[W - 2] = sc[u];
    }
  }
  // the tile that ends the row leaves the last W-1 inputs in its window
  if (a.final_states && t1 == a.T) {
#pragma unroll
    for (int j = 0; j < W - 1; ++j) {
#pragma unroll
      for (int c = 0; c < N; ++c)
        ste<DT>(a.final_states, ((long long)b * a.D + d0 + c) * (W - 1) + j, win[j][c]);
    }
  }
}

// Time-contiguous layout (x_st == o_st == 1): lane = VEC consecutive time
// steps of one (b, d) row; the W-1 inputs before a lane's first step come
// from the previous lane (shuffle) or, for lane 0, from memory.
template <int DT, int W>
__global__ __launch_bounds__(256) void conv1d_tc_kernel(ConvArgs a) {
  constexpr int N = Elt<DT>::VEC;
  const int d = blockIdx.y, b = blockIdx.z;
  const int t0 = (blockIdx.x * 256 + threadIdx.x) * N;
  const int lane = threadIdx.x % 64;
  float w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = ldp(a.weight, (long long)d * W + j, a.wdt);
  const float bs = a.bias ? ldp(a.bias, d, a.wdt) : 0.f;
  const long long xr = (long long)b * a.x_sb + (long long)d * a.x_sd;
  const long long orow = (long long)b * a.o_sb + (long long)d * a.o_sd;
  const bool full = t0 + N <= a.T;
  float cur[N];
  if (full) {
    ldv<DT>(a.x, xr + t0, cur);
  } else {
#pragma unroll
    for (int c = 0; c < N; ++c) cur[c] = (t0 + c < a.T) ? lde<DT>(a.x, xr + t0 + c) : 0.f;
  }
  float prev[W - 1];
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const float up = __shfl_up(cur[N - (W - 1) + j], 1);
    const int p = t0 - (W - 1) + j;
    prev[j] = lane > 0 ? up : ((p >= 0 && p < a.T) ? lde<DT>(a.x, xr + p) : 0.f);
  }
  if (t0 >= a.T) return;
  float acc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float s = bs;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int m = i - (W - 1) + j;
      s += w[j] * (m >= 0 ? cur[m] : prev[(W - 1) + m]);
    }
    acc[i] = a.silu ? silu_f(s) : s;
  }
  if (full) {
    stv<DT>(a.out, orow + t0, acc);
  } else {
#pragma unroll
    for (int c = 0; c < N; ++c)
      if (t0 + c < a.T) ste<DT>(a.out, orow + t0 + c, acc[c]);
  }
}

// Any other strides: one lane per output element, window read directly.
template <int DT, int W>
__global__ __launch_bounds__(256) void conv1d_any_kernel(ConvArgs a) {
  const long long n = (long long)a.B * a.D * a.T;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int t = (int)(i % a.T);
    const int d = (int)((i / a.T) % a.D);
    const int b = (int)(i / ((long long)a.T * a.D));
    const long long xr = (long long)b * a.x_sb + (long long)d * a.x_sd;
    const int32_t* sq = a.seq_idx ? a.seq_idx + (long long)b * a.T : nullptr;
    const int st = sq ? sq[t] : 0;
    float s = a.bias ? ldp(a.bias, d, a.wdt) : 0.f;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int p = t - (W - 1) + j;
      float xv = 0.f;
      if (p >= 0) {
        if (!sq || sq[p] == st) xv = lde<DT>(a.x, xr + p * a.x_st);
      } else if (a.init && !sq) {
        xv = lde<DT>(a.init, ((long long)b * a.D + d) * (W - 1) + (W - 1) + p);
      }
      s += ldp(a.weight, (long long)d * W + j, a.wdt) * xv;
    }
    ste<DT>(a.out, (long long)b * a.o_sb + (long long)d * a.o_sd + (long long)t * a.o_st,
            a.silu ? silu_f(s) : s);
    if (a.final_states && t == a.T - 1) {
#pragma unroll
      for (int j = 0; j < W - 1; ++j) {
        const int p = a.T - (W - 1) + j;
        float xv = 0.f;
        if (p >= 0) xv = lde<DT>(a.x, xr + p * a.x_st);
        else if (a.init) xv = lde<DT>(a.init, ((long long)b * a.D + d) * (W - 1) + (W - 1) + p);
        ste<DT>(a.final_states, ((long long)b * a.D + d) * (W - 1) + j, xv);
      }
    }
  }
}

// Rows with T == 0 still owe their final states (the initial states, or 0).
template <int DT, int W>
__global__ __launch_bounds__(256) void conv1d_empty_final_kernel(ConvArgs a) {
  const long long n = (long long)a.B * a.D * (W - 1);
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  ste<DT>(a.final_states, i, a.init ? lde<DT>(a.init, i) : 0.f);
}

// ------------------------------------------------ causal conv1d update ----
// One lane per (batch row, channel): the S state inputs are read once into
// registers, the L new outputs computed, then the state is rewritten.
template <int DT>
__global__ __launch_bounds__(256) void conv1d_update_kernel(
    const void* x, void* state, const void* weight, const void* bias, const int32_t* idx,
    void* out, int D, int L, int W, int S, int num_slots, long long x_sb, long long x_sd,
    long long x_st, long long o_sb, long long o_sd, long long o_st, int silu, int wdt) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (d >= D) return;
  const int slot = idx ? idx[b] : b;
  if (slot < 0 || slot >= num_slots) return;
  const long long sb = ((long long)slot * D + d) * S;
  float sv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) sv[i] = i < S ? lde<DT>(state, sb + i) : 0.f;
  float w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = j < W ? ldp(weight, (long long)d * W + j, wdt) : 0.f;
  const float bs = bias ? ldp(bias, d, wdt) : 0.f;
  const long long xr = (long long)b * x_sb + (long long)d * x_sd;
  // window position p in [0, S + L): state element p, then input p - S
  auto win = [&](int p) -> float {
    if (p >= S) return lde<DT>(x, xr + (long long)(p - S) * x_st);
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) v = (p == i) ? sv[i] : v;
    return v;
  };
  for (int t = 0; t < L; ++t) {
    float s = bs;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < W) s += w[j] * win(S + t - (W - 1) + j);
    ste<DT>(out, (long long)b * o_sb + (long long)d * o_sd + (long long)t * o_st,
            silu ? silu_f(s) : s);
  }
  float ns[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ns[i] = i < S ? win(L + i) : 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < S) ste<DT>(state, sb + i, ns[i]);
}

// Channel-contiguous inputs (x_sd == o_sd == 1): lane = VEC consecutive
// channels; their S state inputs are VEC * S consecutive elements (S 16-byte
// loads), the inputs of one token one 16-byte load.  The last S inputs are
// kept in registers while the L new tokens stream through.
template <int DT, int W, int S>
__device__ __forceinline__ void conv_update_row(const void* x, void* state, void* out,
                                                long long sb, long long xr, long long orow,
                                                int L, long long x_st, long long o_st,
                                                const float (&wf)[Elt<DT>::VEC * W],
                                                const float (&bs)[Elt<DT>::VEC], int silu) {
  constexpr int N = Elt<DT>::VEC;
  float raw[N * S];
#pragma unroll
  for (int v = 0; v < S; ++v) {
    float tmp[N];
    ldv<DT>(state, sb + v * N, tmp);
#pragma unroll
    for (int k = 0; k < N; ++k) raw[v * N + k] = tmp[k];
  }
  float hist[S][N];   // hist[i][c]: the i-th oldest kept input of channel c
#pragma unroll
  for (int i = 0; i < S; ++i) {
#pragma unroll
    for (int c = 0; c < N; ++c) hist[i][c] = raw[c * S + i];
  }
  for (int t = 0; t < L; ++t) {
    float cur[N];
    ldv<DT>(x, xr + t * x_st, cur);
    float acc[N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
      float v = bs[c] + wf[c * W + W - 1] * cur[c];
#pragma unroll
      for (int j = 0; j < W - 1; ++j) v += wf[c * W + j] * hist[S - (W - 1) + j][c];
      acc[c] = silu ? silu_f(v) : v;
    }
    stv<DT>(out, orow + t * o_st, acc);
#pragma unroll
    for (int i = 0; i + 1 < S; ++i) {
#pragma unroll
      for (int c = 0; c < N; ++c) hist[i][c] = hist[i + 1][c];
    }
#pragma unroll
    for (int c = 0; c < N; ++c) hist[S - 1][c] = cur[c];
  }
#pragma unroll
  for (int v = 0; v < S; ++v) {
    float tmp[N];
#pragma unroll
    for (int k = 0; k < N; ++k) tmp[k] = hist[(v * N + k) % S][(v * N + k) / S];
    stv<DT>(state, sb + v * N, tmp);
  }
}

// One batch row per lane (RB rows would share one load of the lane's
// weights, but 4 rows per lane leave too few lanes at decode sizes).
template <int DT, int W, int S>
__global__ __launch_bounds__(256) void conv1d_update_vec_kernel(
    const void* x, void* state, const void* weight, const void* bias, const int32_t* idx,
    void* out, int B, int D, int L, int num_slots, long long x_sb, long long x_st,
    long long o_sb, long long o_st, int silu, int wdt) {
  constexpr int N = Elt<DT>::VEC;
  constexpr int RB = 1;
  const int d0 = (blockIdx.x * 256 + threadIdx.x) * N;
  if (d0 >= D) return;
  float wf[N * W], bs[N];
  ld_params<N * W>(weight, (long long)d0 * W, wdt, wf);
  if (bias) {
    ld_params<N>(bias, d0, wdt, bs);
  } else {
#pragma unroll
    for (int c = 0; c < N; ++c) bs[c] = 0.f;
  }
  const int b1 = min(B, (int)(blockIdx.y + 1) * RB);
  for (int b = blockIdx.y * RB; b < b1; ++b) {
    const int slot = idx ? idx[b] : b;
    if (slot < 0 || slot >= num_slots) continue;
    conv_update_row<DT, W, S>(x, state, out, ((long long)slot * D + d0) * S,
                              (long long)b * x_sb + d0, (long long)b * o_sb + d0, L, x_st, o_st,
                              wf, bs, silu);
  }
}

}  // namespace gdn

// ------------------------------------------------------------- host ----
using gdn::dtype_ok;

namespace {

int esize(int dt) { return dt == GDN_DTYPE_F32 ? 4 : 2; }
int vec_of(int dt) { return dt == GDN_DTYPE_F32 ? 4 : 8; }
unsigned grid_for(long long n, int per_block) {
  long long g = (n + per_block - 1) / per_block;
  return (unsigned)(g < 1 ? 1 : (g > 65535LL * 16 ? 65535LL * 16 : g));
}

}  // namespace

extern "C" int gdn_gating_fwd(const void* A_log, const void* a, const void* b,
                              const void* dt_bias, float* g, float* beta, long long rows, int H,
                              int a_dtype, int b_dtype, int p_dtype, float sp_beta,
                              float sp_threshold, void* stream) {
  if (rows < 0 || H <= 0) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_gating_fwd: rows >= 0, H > 0");
  if (!dtype_ok(a_dtype) || !dtype_ok(b_dtype) || !dtype_ok(p_dtype))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_gating_fwd: unsupported dtype code");
  if (!(sp_beta > 0.f)) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_gating_fwd: softplus beta must be > 0");
  const long long n = rows * H;
  if (n == 0) return GDN_OK;
  gdn_host::launch_begin();
  if (!A_log || !a || !dt_bias || !g || (beta && !b))
    return gdn_host::fail(GDN_ERR_NULL, "gdn_gating_fwd: A_log, a, dt_bias, g (and b with beta) must be non-NULL");
  const gdn::GateIn gp{A_log, a, beta ? b : nullptr, dt_bias, a_dtype, b_dtype, p_dtype, sp_beta,
                       sp_threshold, n, H};
  hipLaunchKernelGGL(gdn::gating_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), gp, g, beta, n, H);
  return gdn_host::check_launch("gdn_gating_fwd");
}

// rows per block of the gating backward: 64, more when that would leave
// over 1024 block partials to sum
static int gating_bwd_rows(long long rows) {
  const long long r = (rows + 1023) / 1024;
  return (int)(r < 64 ? 64 : r);
}
static long long gating_bwd_blocks(long long rows) {
  const int R = gating_bwd_rows(rows);
  return (rows + R - 1) / R;
}

extern "C" size_t gdn_gating_bwd_workspace_bytes(long long rows, int H) {
  if (rows < 0 || H <= 0) return 0;
  return (size_t)gating_bwd_blocks(rows) * (size_t)H * 2 * sizeof(float);
}

extern "C" int gdn_gating_bwd(const void* A_log, const void* a, const void* b,
                              const void* dt_bias, const float* dg, const float* dbeta,
                              void* dA_log, void* da, void* db, void* ddt_bias, long long rows,
                              int H, int a_dtype, int b_dtype, int p_dtype, float sp_beta,
                              float sp_threshold, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (rows < 0 || H <= 0 || H > 256)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_gating_bwd: rows >= 0 and 0 < H <= 256");
  if (!dtype_ok(a_dtype) || !dtype_ok(b_dtype) || !dtype_ok(p_dtype))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_gating_bwd: unsupported dtype code");
  if (!(sp_beta > 0.f)) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_gating_bwd: softplus beta must be > 0");
  if (!A_log || !dt_bias || (rows > 0 && (!a || !dg || !da)))
    return gdn_host::fail(GDN_ERR_NULL, "gdn_gating_bwd: A_log, dt_bias, a, dg and da must be non-NULL");
  if ((db != nullptr) != (dbeta != nullptr) || (db && rows > 0 && !b))
    return gdn_host::fail(GDN_ERR_NULL, "gdn_gating_bwd: db and dbeta go together, and need b");
  const long long nblk = gating_bwd_blocks(rows);
  const size_t need = gdn_gating_bwd_workspace_bytes(rows, H);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return gdn_host::fail(GDN_ERR_WORKSPACE, "gdn_gating_bwd: workspace NULL or smaller than "
                                             "gdn_gating_bwd_workspace_bytes(rows, H)");
  if (!dA_log && !ddt_bias && rows == 0) return GDN_OK;
  gdn_host::launch_begin();
  const hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  if (rows > 0) {
    const gdn::GateIn gp{A_log, a, b, dt_bias, a_dtype, b_dtype, p_dtype, sp_beta, sp_threshold,
                         rows * H, H};
    hipLaunchKernelGGL(gdn::gating_bwd_kernel, dim3((unsigned)nblk), dim3(256), 0, st, gp, dg,
                       dbeta, da, db, part, rows, H, gating_bwd_rows(rows));
  }
  if (dA_log || ddt_bias)
    hipLaunchKernelGGL(gdn::gating_bwd_reduce_kernel, dim3((H + 255) / 256), dim3(256), 0, st,
                       part, (int)nblk, H, dA_log, ddt_bias, p_dtype);
  return gdn_host::check_launch("gdn_gating_bwd");
}

extern "C" int gdn_l2norm_fwd(const void* x, void* y, long long rows, int D, float eps,
                              int dtype, void* stream) {
  if (rows < 0) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_l2norm_fwd: rows must be >= 0");
  if (!(D == 64 || D == 128 || D == 256))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_l2norm_fwd: D must be 64, 128 or 256");
  if (!dtype_ok(dtype)) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_l2norm_fwd: unsupported dtype code");
  if (rows == 0) return GDN_OK;
  gdn_host::launch_begin();
  if (!x || !y) return gdn_host::fail(GDN_ERR_NULL, "gdn_l2norm_fwd: x and y must be non-NULL");
  if (rows > (1LL << 36)) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_l2norm_fwd: too many rows");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_l2norm_fwd: x and y must be 16-byte aligned");
  auto st = static_cast<hipStream_t>(stream);
#define GDN_L2(DD, TT)                                                                         \
  if (D == DD && dtype == TT) {                                                                \
    constexpr int RPB = gdn::RowShape<DD, TT>::RPB;                                            \
    hipLaunchKernelGGL((gdn::l2norm_kernel<DD, TT>), dim3((unsigned)((rows + RPB - 1) / RPB)), \
                       dim3(256), 0, st, x, y, rows, eps);                                     \
    return gdn_host::check_launch("gdn_l2norm_fwd");                                           \
  }
  GDN_L2(64, GDN_DTYPE_F32) GDN_L2(64, GDN_DTYPE_BF16) GDN_L2(64, GDN_DTYPE_F16)
  GDN_L2(128, GDN_DTYPE_F32) GDN_L2(128, GDN_DTYPE_BF16) GDN_L2(128, GDN_DTYPE_F16)
  GDN_L2(256, GDN_DTYPE_F32) GDN_L2(256, GDN_DTYPE_BF16) GDN_L2(256, GDN_DTYPE_F16)
#undef GDN_L2
  return gdn_host::fail(GDN_ERR_SHAPE, "gdn_l2norm_fwd: unsupported configuration");
}

extern "C" int gdn_rmsnorm_gated_fwd(const void* x, const void* z, const void* weight, void* out,
                                     long long rows, int D, float eps, int dtype, int w_dtype,
                                     void* stream) {
  if (rows < 0) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_rmsnorm_gated_fwd: rows must be >= 0");
  if (!(D == 64 || D == 128 || D == 256))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_rmsnorm_gated_fwd: D must be 64, 128 or 256");
  if (!dtype_ok(dtype) || !dtype_ok(w_dtype))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_rmsnorm_gated_fwd: unsupported dtype code");
  if (rows == 0) return GDN_OK;
  gdn_host::launch_begin();
  if (!x || !z || !weight || !out)
    return gdn_host::fail(GDN_ERR_NULL, "gdn_rmsnorm_gated_fwd: x, z, weight and out must be non-NULL");
  if (rows > (1LL << 36)) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_rmsnorm_gated_fwd: too many rows");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(z) |
       reinterpret_cast<uintptr_t>(out)) % 16)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_rmsnorm_gated_fwd: x, z and out must be 16-byte aligned");
  auto st = static_cast<hipStream_t>(stream);
#define GDN_RN(DD, TT)                                                                         \
  if (D == DD && dtype == TT) {                                                                \
    constexpr int RPB = gdn::RowShape<DD, TT>::RPB;                                            \
    hipLaunchKernelGGL((gdn::rmsnorm_gated_kernel<DD, TT>),                                    \
                       dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, st, x, z,       \
                       weight, out, rows, eps, w_dtype);                                       \
    return gdn_host::check_launch("gdn_rmsnorm_gated_fwd");                                    \
  }
  GDN_RN(64, GDN_DTYPE_F32) GDN_RN(64, GDN_DTYPE_BF16) GDN_RN(64, GDN_DTYPE_F16)
  GDN_RN(128, GDN_DTYPE_F32) GDN_RN(128, GDN_DTYPE_BF16) GDN_RN(128, GDN_DTYPE_F16)
  GDN_RN(256, GDN_DTYPE_F32) GDN_RN(256, GDN_DTYPE_BF16) GDN_RN(256, GDN_DTYPE_F16)
#undef GDN_RN
  return gdn_host::fail(GDN_ERR_SHAPE, "gdn_rmsnorm_gated_fwd: unsupported configuration");
}

namespace {

template <int DT, int W>
int launch_conv(const gdn::ConvArgs& a, hipStream_t st) {
  const int N = vec_of(DT);
  const bool vec_aligned_x = (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
  const bool vec_aligned_o = (reinterpret_cast<uintptr_t>(a.out) % 16) == 0;
  const bool vec_aligned_w = ((reinterpret_cast<uintptr_t>(a.weight) |
                               reinterpret_cast<uintptr_t>(a.bias)) % 16) == 0;
  if (a.T == 0) {
    if (a.final_states) {
      const long long n = (long long)a.B * a.D * (W - 1);
      hipLaunchKernelGGL((gdn::conv1d_empty_final_kernel<DT, W>), dim3(grid_for(n, 256)),
                         dim3(256), 0, st, a);
    }
    return gdn_host::check_launch("gdn_causal_conv1d_fwd");
  }
  if (a.x_sd == 1 && a.o_sd == 1 && a.D % N == 0 && a.x_sb % N == 0 && a.x_st % N == 0 &&
      a.o_sb % N == 0 && a.o_st % N == 0 && vec_aligned_x && vec_aligned_o && vec_aligned_w) {
    const int TT = 64;   // halo re-reads (W-1 rows per tile) miss L2: keep tiles long
    const dim3 grid((unsigned)((a.D / N + 255) / 256), (unsigned)((a.T + TT - 1) / TT),
                    (unsigned)a.B);
    hipLaunchKernelGGL((gdn::conv1d_cl_kernel<DT, W>), grid, dim3(256), 0, st, a, TT);
  } else if (a.x_st == 1 && a.o_st == 1 && !a.seq_idx && !a.init && !a.final_states &&
             a.x_sb % N == 0 && a.x_sd % N == 0 && a.o_sb % N == 0 && a.o_sd % N == 0 &&
             vec_aligned_x && vec_aligned_o) {
    const dim3 grid((unsigned)((a.T + 256 * N - 1) / (256 * N)), (unsigned)a.D, (unsigned)a.B);
    hipLaunchKernelGGL((gdn::conv1d_tc_kernel<DT, W>), grid, dim3(256), 0, st, a);
  } else {
    const long long n = (long long)a.B * a.D * a.T;
    hipLaunchKernelGGL((gdn::conv1d_any_kernel<DT, W>), dim3(grid_for(n, 256)), dim3(256), 0,
                       st, a);
  }
  return gdn_host::check_launch("gdn_causal_conv1d_fwd");
}

}  // namespace

extern "C" int gdn_causal_conv1d_fwd(const void* x, const void* weight, const void* bias,
                                     const int32_t* seq_idx, const void* initial_states,
                                     void* final_states, void* out, int B, int D, int T, int W,
                                     long long x_sb, long long x_sd, long long x_st,
                                     long long o_sb, long long o_sd, long long o_st, int silu,
                                     int dtype, int w_dtype, void* stream) {
  if (B < 0 || D < 0 || T < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_fwd: sizes must be >= 0");
  if (W < 2 || W > 4) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_fwd: W must be 2, 3 or 4");
  if (!dtype_ok(dtype) || !dtype_ok(w_dtype))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_fwd: unsupported dtype code");
  if (x_sb < 0 || x_sd < 0 || x_st < 0 || o_sb < 0 || o_sd < 0 || o_st < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_fwd: strides must be >= 0");
  if (seq_idx && initial_states)
    return gdn_host::fail(GDN_ERR_SHAPE,
                          "gdn_causal_conv1d_fwd: seq_idx and initial_states cannot be combined");
  if ((long long)B * D == 0) return GDN_OK;
  gdn_host::launch_begin();
  if (!weight || (T > 0 && (!x || !out)))
    return gdn_host::fail(GDN_ERR_NULL, "gdn_causal_conv1d_fwd: x, weight and out must be non-NULL");
  if ((long long)B * D * (long long)(T > 0 ? T : 1) > (1LL << 40) || D > (1 << 24))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_fwd: problem too large");
  if (T > 0 && x == out)
    return gdn_host::fail(GDN_ERR_ALIAS, "gdn_causal_conv1d_fwd: out must not alias x");
  const gdn::ConvArgs a{x, weight, bias, seq_idx, initial_states, final_states, out, B, D, T,
                        x_sb, x_sd, x_st, o_sb, o_sd, o_st, silu, w_dtype};
  auto st = static_cast<hipStream_t>(stream);
#define GDN_CV(TT, WW) \
  if (dtype == TT && W == WW) return launch_conv<TT, WW>(a, st);
  GDN_CV(GDN_DTYPE_F32, 2) GDN_CV(GDN_DTYPE_F32, 3) GDN_CV(GDN_DTYPE_F32, 4)
  GDN_CV(GDN_DTYPE_BF16, 2) GDN_CV(GDN_DTYPE_BF16, 3) GDN_CV(GDN_DTYPE_BF16, 4)
  GDN_CV(GDN_DTYPE_F16, 2) GDN_CV(GDN_DTYPE_F16, 3) GDN_CV(GDN_DTYPE_F16, 4)
#undef GDN_CV
  return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_fwd: unsupported configuration");
}

extern "C" int gdn_causal_conv1d_update(const void* x, void* conv_state, const void* weight,
                                        const void* bias, const int32_t* conv_state_indices,
                                        void* out, int B, int D, int L, int W, int S,
                                        int num_slots, long long x_sb, long long x_sd,
                                        long long x_st, long long o_sb, long long o_sd,
                                        long long o_st, int silu, int dtype, int w_dtype,
                                        void* stream) {
  if (B < 0 || D < 0 || num_slots < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: sizes must be >= 0");
  if (W < 2 || W > 4) return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: W must be 2, 3 or 4");
  if (S < W - 1 || S > 8)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: state length must be in [W-1, 8]");
  if (L < 1 || L > 64)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: tokens per row must be in [1, 64]");
  if (!dtype_ok(dtype) || !dtype_ok(w_dtype))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: unsupported dtype code");
  if (x_sb < 0 || x_sd < 0 || x_st < 0 || o_sb < 0 || o_sd < 0 || o_st < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: strides must be >= 0");
  if (!conv_state_indices && num_slots < B)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: without indices num_slots must be >= B");
  if ((long long)B * D == 0) return GDN_OK;
  gdn_host::launch_begin();
  if (!x || !conv_state || !weight || !out)
    return gdn_host::fail(GDN_ERR_NULL, "gdn_causal_conv1d_update: x, conv_state, weight and out must be non-NULL");
  if (B > 65535 || D > (1 << 24))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: problem too large");
  auto st = static_cast<hipStream_t>(stream);
  const int N = vec_of(dtype);
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                          reinterpret_cast<uintptr_t>(conv_state) |
                          reinterpret_cast<uintptr_t>(weight) |
                          reinterpret_cast<uintptr_t>(bias);
  // the token stride only matters for L > 1
  const bool st_ok = L == 1 || (x_st % N == 0 && o_st % N == 0);
  if (x_sd == 1 && o_sd == 1 && D % N == 0 && x_sb % N == 0 && o_sb % N == 0 && st_ok &&
      align % 16 == 0 && (S == W - 1 || S == W)) {
    const dim3 vgrid((unsigned)((D / N + 255) / 256), (unsigned)B);
#define GDN_CUV(TT, WW, SS)                                                                    \
    if (dtype == TT && W == WW && S == SS) {                                                   \
      hipLaunchKernelGGL((gdn::conv1d_update_vec_kernel<TT, WW, SS>), vgrid, dim3(256), 0, st, \
                         x, conv_state, weight, bias, conv_state_indices, out, B, D, L,        \
                         num_slots, x_sb, x_st, o_sb, o_st, silu, w_dtype);                    \
      return gdn_host::check_launch("gdn_causal_conv1d_update");                               \
    }
#define GDN_CUV_W(TT) \
    GDN_CUV(TT, 2, 1) GDN_CUV(TT, 2, 2) GDN_CUV(TT, 3, 2) GDN_CUV(TT, 3, 3) GDN_CUV(TT, 4, 3) GDN_CUV(TT, 4, 4)
    GDN_CUV_W(GDN_DTYPE_F32) GDN_CUV_W(GDN_DTYPE_BF16) GDN_CUV_W(GDN_DTYPE_F16)
#undef GDN_CUV_W
#undef GDN_CUV
  }
  const dim3 grid((unsigned)((D + 255) / 256), (unsigned)B);
#define GDN_CU(TT)                                                                              \
  if (dtype == TT) {                                                                            \
    hipLaunchKernelGGL((gdn::conv1d_update_kernel<TT>), grid, dim3(256), 0, st, x, conv_state,  \
                       weight, bias, conv_state_indices, out, D, L, W, S, num_slots, x_sb,      \
                       x_sd, x_st, o_sb, o_sd, o_st, silu, w_dtype);                            \
    return gdn_host::check_launch("gdn_causal_conv1d_update");                                  \
  }
  GDN_CU(GDN_DTYPE_F32) GDN_CU(GDN_DTYPE_BF16) GDN_CU(GDN_DTYPE_F16)
#undef GDN_CU
  return gdn_host::fail(GDN_ERR_SHAPE, "gdn_causal_conv1d_update: unsupported configuration");
}
