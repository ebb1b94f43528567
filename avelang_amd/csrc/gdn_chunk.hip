// Chunked gated-delta-rule prefill for gfx950 (chunk = 64 tokens).
//
// Operator semantics: transformers modeling_qwen3_next.py:374-453
// (torch_chunk_gated_delta_rule); the reference repository has no GDN code,
// its launcher convention is python/avelang/backends/amdgpu/driver.py:324-343.
//
// Per chunk c of one sequence and v-head h (rows i, j in [0, 64)):
//   G     = cumsum(g)                  Gam_ij = exp(G_i - G_j), i >= j
//   A     = strict_lower(diag(beta) K K^T * Gam)
//   Tb    = (I + A)^-1 diag(beta)
//   P     = scale * lower_incl(Q K^T * Gam)
// and, carried across chunks with the fp32 state S [K][V]:
//   Y     = V - e^G * (K S)            (so vnew = u - w S = Tb Y)
//   vnew  = Tb Y
//   o     = scale * e^G * (Q S) + P vnew
//   S     = e^G_L S + K^T (e^(G_L - G) * vnew)
//
// Three launches:
//   chunk_table_kernel  sequence -> first-chunk offsets (varlen plumbing)
//   chunk_prep_kernel   one workgroup per (chunk, v-head), fully parallel:
//                       K K^T and Q K^T on MFMA, blocked UT inverse in fp32,
//                       Tb and P written as ready-made fp16 MFMA A-operand
//                       fragments, the chunk's K and Q as fp16 copies laid
//                       out for the chain
//   chunk_chain_sw_kernel (gdn_chunk_chain.hip)  one workgroup per (sequence,
//                       v-head, 16-column V tile), sequential over that
//                       sequence's chunks; one wave holds the fp32 state slice
//                       in VGPRs for the whole sequence, every product is a
//                       16x16x32 fp16 MFMA, and two more waves stage operands
//                       and form the output.
// Precision: every chain product takes fp16 operands rounded from fp32 (one
// MFMA pass each; fp16's 11-bit significand keeps the final state within
// ~4e-4 relative Frobenius at any sequence length, against ~3e-3 for single
// bf16).  Operands stay far inside fp16's range for l2-normalised q / k and
// v of the magnitudes a layer produces.
#include <mutex>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

// -------------------------------------------------------- chunk table ----
// Sequence -> first-chunk offsets, after checking the cu_seqlens contract
// (cu[0] == 0, non-decreasing, cu[N] == total).  A violation is recorded in
// *status and every sequence is then treated as empty (all offsets 0), so
// that no later kernel reads or writes past the packed tokens; the caller's
// outputs are zero-filled by zero_on_violation_kernel.
__global__ __launch_bounds__(256) void chunk_table_kernel(const int32_t* __restrict__ cu,
                                                          int N, int T, int total,
                                                          int ncmax, int32_t* __restrict__ off,
                                                          int32_t* __restrict__ status) {
  __shared__ int part[257];
  __shared__ int bad;
  const int tid = threadIdx.x;
  const int per = (N + 255) / 256;
  const int a = min(tid * per, N), b = min(a + per, N);
  if (tid == 0) bad = cu[0] != 0 ? 1 : (cu[N] != total ? 3 : 0);
  __syncthreads();
  for (int n = a; n < b; ++n)
    if (cu[n + 1] < cu[n]) atomicMax(&bad, 2);
  __syncthreads();
  if (bad) {
    for (int n = tid; n <= N; n += 256) off[n] = 0;
    if (tid == 0) *status = bad;
    return;
  }
  if (tid == 0) *status = 0;
  int sum = 0;
  for (int n = a; n < b; ++n) {
    int s, e;
    seq_bounds(cu, n, T, total, s, e);
    sum += (e - s + kChunk - 1) / kChunk;
  }
  part[tid + 1] = sum;
  __syncthreads();
  if (tid == 0) {
    part[0] = 0;
    for (int i = 1; i <= 256; ++i) part[i] += part[i - 1];
  }
  __syncthreads();
  int run = part[tid];
  for (int n = a; n < b; ++n) {
    off[n] = min(run, ncmax);
    int s, e;
    seq_bounds(cu, n, T, total, s, e);
    run += (e - s + kChunk - 1) / kChunk;
  }
  if (tid == 255) off[N] = min(part[256], ncmax);
}

__global__ __launch_bounds__(256) void zero_on_violation_kernel(const int32_t* __restrict__ status,
                                                                ZeroList z) {
  if (*status == 0) return;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (int i = 0; i < 5; ++i) {
    // 16-byte stores over the 16-byte-aligned body, then the tail bytes
    unsigned char* p = static_cast<unsigned char*>(z.p[i]);
    if (!p) continue;
    const size_t n = z.bytes[i];
    const size_t head = (16 - ((uintptr_t)p & 15)) & 15;
    const size_t h = head < n ? head : n;
    const size_t body = (n - h) / 16;
    for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < body; j += stride)
      reinterpret_cast<uint4*>(p + h)[j] = uint4{0, 0, 0, 0};
    for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < h + (n - h - 16 * body);
         j += stride)
      p[j < h ? j : h + 16 * body + (j - h)] = 0;
  }
}

void launch_zero_on_violation(const int32_t* status, const ZeroList& z, hipStream_t st) {
  hipLaunchKernelGGL(zero_on_violation_kernel, dim3(256), dim3(256), 0, st, status, z);
}

// ---------------------------------------------------------- prep (K1) ----
constexpr int kLdA = 68;   // fp32 row stride of A / Tm in LDS (rows 16-byte aligned)

// Inclusive prefix sum over the 64 lanes as DPP moves: within each 16-lane
// row by shifts to the right (lanes before the row's start read 0), then
// the last lane of row 0 and of row 2 is added to rows 1 and 3 (row_bcast15)
// and the last lane of row 1 to rows 2 and 3 (row_bcast31).
__device__ __forceinline__ float prefix_sum64(float x) {
  auto shr = [](float v, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                decltype(ctrl)::value, 0xF, 0xF,
                                                                true));
  };
  x += shr(x, std::integral_constant<int, 0x111>{});
  x += shr(x, std::integral_constant<int, 0x112>{});
  x += shr(x, std::integral_constant<int, 0x114>{});
  x += shr(x, std::integral_constant<int, 0x118>{});
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142,
                                                             0xA, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x143,
                                                             0xC, 0xF, false));
  return x;
}

// Rows of MFMA fragments scaled by r and rounded back to bf16.
template <int KB>
__device__ __forceinline__ void scale_frags(u16x8 (&f)[KB], float r) {
#pragma unroll
  for (int b = 0; b < KB; ++b) {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[b][i] = f2bf(bf2f(f[b][i]) * r);
  }
}

// One workgroup per (chunk, v-head).  Wave w owns chunk rows 16w..16w+15.
// BWD (the backward's recomputation) also writes T itself and the A-operand
// fragments of Tb^T and P^T for the reverse chain.  OUT: the chain forms the
// output, and so reads the P fragments (the backward's recomputation does
// not).  L2: use_qk_l2norm (a compile-time flag: with one code path per form
// the compiler's waits for the K / Q row loads never include the normalised
// rows' stores).
template <int K, bool BWD, bool OUT, bool L2>
__global__ __launch_bounds__(256) void chunk_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const float* __restrict__ g, const float* __restrict__ beta,
    const int32_t* __restrict__ cu, int N, int T, int total, int Hqk, int Hv, float scale,
    ChunkWs ws, GateIn gate) {
  constexpr int KB = K / 32;
  // strictly lower 16 x 16 blocks of A only (block (bi, m), m < bi, at
  // bi (bi - 1) / 2 + m; row stride 20 keeps float4 rows aligned and the 16
  // rows of a read on distinct banks): 7.5 KB instead of a full 64 x 68
  // array, which lets 5 workgroups share a CU instead of 4
  __shared__ __attribute__((aligned(16))) float Ab[6][16][20];
  __shared__ __attribute__((aligned(16))) float Tm[64 * kLdA];
  // The chunk's K rows are staged in Tm's space until K K^T is formed.
  static_assert(64 * (K + 8) * 2 <= 64 * kLdA * 4, "K staging must fit in Tm");
  uint16_t (*Ks)[K + 8] = reinterpret_cast<uint16_t (*)[K + 8]>(Tm);
  // diagonal blocks of A, transposed (column j of block w is AdT[w][j])
  __shared__ __attribute__((aligned(16))) float AdT[4][16][16];
  __shared__ __attribute__((aligned(16))) float Bs[64];
  __shared__ __attribute__((aligned(16))) float Gs[64];
  // P (bf16, row-major) for the P^T fragments (backward only)
  __shared__ __attribute__((aligned(16))) uint16_t Ps[BWD ? 64 : 1][72];

  const int ci = blockIdx.x;
  const int h = blockIdx.y;
  int n, cfirst;
  if (cu) {
    const int32_t* off = ws.off;
    if (ci >= off[N]) return;
    // sequence owning chunk ci: largest n < N with off[n] <= ci
    int lo = 0, hi = N;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= ci) lo = mid; else hi = mid;
    }
    n = lo;
    cfirst = off[n];
  } else {
    // equal-length sequences: the chunk table is arithmetic
    const int nct = (T + kChunk - 1) / kChunk;
    n = ci / nct;
    cfirst = n * nct;
  }
  int s, e;
  seq_bounds(cu, n, T, total, s, e);
  const int t0 = s + (ci - cfirst) * kChunk;
  const int L = min(kChunk, e - t0);
  const int hq = h / (Hv / Hqk);

  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const int r16 = lane % 16, grp = lane / 16;

  // g and beta of the chunk's rows (wave 0), issued first so that their
  // latency overlaps that of the K / Q rows rather than following it.  With
  // the gating computed here (gate.a set) only its raw loads go out now; its
  // math (gate_eval: the values gate_at gives) waits until the K / Q row
  // loads are in flight too.
  float gv = 0.f, bv = 0.f;
  GateRaw graw{};
  if (w == 0) {
    const size_t grow = (size_t)(t0 + min(lane, L - 1)) * Hv + h;
    if (gate.a) {
      graw = gate_load(gate, (long long)grow, h);
    } else {
      gv = g[grow];
      bv = beta[grow];
    }
  }
  // K / Q rows straight into MFMA fragments (this wave's rows); the K rows
  // are also staged in LDS, where the other waves read them as B operands.
  // Padding rows (row >= L) repeat row L-1: their A rows are scaled by
  // beta = 0 and their P entries are never used, so the values only need to
  // be finite, and the loads stay branch-free.
  u16x8 ka[KB], qa[KB];
  {
    const size_t ro = ((size_t)(t0 + min(16 * w + r16, L - 1)) * Hqk + hq) * K + 8 * grp;
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      ka[b] = *reinterpret_cast<const u16x8*>(k + ro + 32 * b);
      qa[b] = *reinterpret_cast<const u16x8*>(q + ro + 32 * b);
    }
    if constexpr (L2) {
      // use_qk_l2norm: a row's K values sit in the 4 lanes r16 + 16 grp; the
      // normalised rows are rounded to bf16 (as a separate l2norm pass would
      // store them), and the first v-head of each qk-head group stores them
      // for the chain (below)
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int b = 0; b < KB; ++b) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xk = bf2f(ka[b][i]), xq = bf2f(qa[b][i]);
          sk += xk * xk;
          sq += xq * xq;
        }
      }
      sk += __shfl_xor(sk, 16);
      sk += __shfl_xor(sk, 32);
      sq += __shfl_xor(sq, 16);
      sq += __shfl_xor(sq, 32);
      const float rk = rsqrtf(sk + 1e-6f), rq = rsqrtf(sq + 1e-6f);
      scale_frags<KB>(ka, rk);
      scale_frags<KB>(qa, rq);
    }
#pragma unroll
    for (int b = 0; b < KB; ++b)
      *reinterpret_cast<u16x8*>(&Ks[16 * w + r16][32 * b + 8 * grp]) = ka[b];
    // The first v-head of each qk-head group stores the chunk's K rows and Q
    // fragments as fp16 for the chain (after the LDS writes above: stores
    // count in the same in-order vector-memory counter as the loads, so a
    // wait for ka ahead of them would also wait for these stores).  K goes
    // in the chain's LDS layout with rows past the sequence end zeroed, so
    // the chain copies it to LDS with contiguous loads; Q as the B-operand
    // fragments the chain's output wave loads (row 16 w + r16, columns
    // 32 b + 8 grp ..).  Not when the plan has no copies (the chain reads
    // the caller's rows).
    if (ws.k16 && h % (Hv / Hqk) == 0) {
      using KL = KLayout<K>;
      const int row = 16 * w + r16;
      unsigned char* kd = ws.k16 + ((size_t)ci * Hqk + hq) * KL::BYTES;
#pragma unroll
      for (int b = 0; b < KB; ++b)
        *reinterpret_cast<u16x8*>(kd + KL::off(row, 4 * b + grp)) =
            row < L ? bf2h8(ka[b]) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (OUT && ws.q16) {
        u16x8* qd = ws.q16 + (((size_t)ci * Hqk + hq) * 4 + w) * KB * 64 + lane;
#pragma unroll
        for (int b = 0; b < KB; ++b) qd[b * 64] = bf2h8(qa[b]);
      }
      // the normalised rows (bf16) for the backward's kernels
      if (L2 && BWD && row < L) {
        const size_t wo = ((size_t)(t0 + row) * Hqk + hq) * K + 8 * grp;
#pragma unroll
        for (int b = 0; b < KB; ++b) {
          *reinterpret_cast<u16x8*>(ws.kn + wo + 32 * b) = ka[b];
          *reinterpret_cast<u16x8*>(ws.qn + wo + 32 * b) = qa[b];
        }
      }
    }
  }
  // gates: wave 0 scans g over the 64 rows (padding rows add 0) and shares
  // G and beta through LDS
  if (w == 0) {
    if (gate.a) gate_eval(gate, graw, gv, bv);
    gv = lane < L ? gv : 0.f;
    bv = lane < L ? bv : 0.f;
    gv = prefix_sum64(gv);
    ws.gate[((size_t)ci * Hv + h) * 64 + lane] = gv;
    Gs[lane] = gv;
    Bs[lane] = bv;
  }
  __syncthreads();

  // Column tiles tc < w are formed transposed, (K K^T)^T and (Q K^T)^T with
  // the staged K rows as the A operand: each lane then holds 4 consecutive
  // columns j of one row i = 16w + r16, so A rows are written as float4 and
  // P goes straight to its fragment slots.  K K^T is symmetric, so the
  // transposed tile is the same product.  The diagonal tile is also formed
  // in the normal orientation for the transposed block AdT.
  //   A = strict_lower(beta_i K K^T Gam), P = scale lower_incl(Q K^T Gam)
  const int i = 16 * w + r16;
  const float Gi = Gs[i], Bi = Bs[i];
  {
    f32x4 kd = zero4();
#pragma unroll
    for (int b = 0; b < KB; ++b) kd = mfma16(ka[b], ka[b], kd);
    const f32x4 Gr = *reinterpret_cast<const f32x4*>(&Gs[16 * w + 4 * grp]);
    const f32x4 Br = *reinterpret_cast<const f32x4*>(&Bs[16 * w + 4 * grp]);
    f32x4 av;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // row 16w + 4grp + r, column i
      av[r] = (i < 16 * w + 4 * grp + r) ? Br[r] * kd[r] * __expf(Gr[r] - Gi) : 0.f;
    }
    *reinterpret_cast<f32x4*>(&AdT[w][r16][4 * grp]) = av;
  }
  u16x8* pdst = ws.pfrag + ((size_t)ci * Hv + h) * 6 * 64;
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int tc = 0; tc < 4; ++tc) {
    f32x4 kt = zero4(), pt = zero4();
    if (tc <= w) {
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const u16x8 kr = *reinterpret_cast<const u16x8*>(&Ks[16 * tc + r16][32 * b + 8 * grp]);
        kt = mfma16(kr, ka[b], kt);
        pt = mfma16(kr, qa[b], pt);
      }
    }
    const f32x4 Gj = *reinterpret_cast<const f32x4*>(&Gs[16 * tc + 4 * grp]);
    f32x4 av, pf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * tc + 4 * grp + r;
      const float gam = (tc <= w && j <= i) ? __expf(Gi - Gj[r]) : 0.f;
      av[r] = (j < i) ? Bi * kt[r] * gam : 0.f;
      pf[r] = scale * pt[r] * gam;
    }
    if (tc < w) *reinterpret_cast<f32x4*>(&Ab[w * (w - 1) / 2 + tc][r16][4 * grp]) = av;
    if constexpr (BWD) *reinterpret_cast<u16x4*>(&Ps[i][16 * tc + 4 * grp]) = f2bf4(pf);
    // P fragment (fp16): slot tb_slot(w, tc / 2), fragment lane
    // r16 + 16 (2 (tc % 2) + grp / 2), elements 4 (grp % 2) .. + 3
    // (k-block 1 of row tiles 0 and 1 is zero and never read: not stored)
    if (OUT && (tc < 2 || w >= 2)) {
      uint16_t* pe = reinterpret_cast<uint16_t*>(
          pdst + tb_slot(w, tc / 2) * 64 + r16 + 16 * (2 * (tc % 2) + grp / 2));
      *reinterpret_cast<u32x2*>(pe + 4 * (grp % 2)) = __builtin_bit_cast(u32x2, f2h4(pf));
    }
  }
  __syncthreads();

  if constexpr (BWD) {
    // fp16 A-operand fragments of Q^T for the reverse chain, in its rho row
    // order: natural key row R = 16 T + r16 is row m = 4 ((R / 8) % 4) + R % 4
    // of rho tile t = 2 (R / 32) + (R / 4) % 2, and lane m + 16 grp of
    // (t, token k-block b) holds Q[32 b + 8 grp + i][R].  Once per qk-head:
    // the chunk's Q rows pass through the K staging space, free after K K^T,
    // and each wave gathers natural key-row tiles w, w + 4, ...
    if (h % (Hv / Hqk) == 0) {
#pragma unroll
      for (int b = 0; b < KB; ++b)
        *reinterpret_cast<u16x8*>(&Ks[16 * w + r16][32 * b + 8 * grp]) = qa[b];
      __syncthreads();
      const size_t qb = ((size_t)ci * Hqk + hq) * (K / 16);
      const int m = 4 * (2 * (w & 1) + (r16 >> 3)) + (r16 & 3);
#pragma unroll
      for (int T = w; T < K / 16; T += 4) {
        const int t = 2 * (T >> 1) + ((r16 >> 2) & 1);
#pragma unroll
        for (int b = 0; b < 2; ++b)
          ws.qtfrag[((qb + t) * 2 + b) * 64 + m + 16 * grp] =
              bf2h8(lds_colfrag(&Ks[0][0], K + 8, 32 * b, 16 * T, lane));
      }
      __syncthreads();
    }
  }

  // (I + A)^-1, blocked by 16.  Diagonal blocks: right-looking elimination,
  // lane c < 16 owns column c (15 dependent levels, not 120).
  if (lane < 16) {
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = (i == lane) ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 15; ++j) {
      float col[16];
#pragma unroll
      for (int i4 = 0; i4 < 16; i4 += 4) {
        const f32x4 c4 = *reinterpret_cast<const f32x4*>(&AdT[w][j][i4]);
        col[i4] = c4[0];
        col[i4 + 1] = c4[1];
        col[i4 + 2] = c4[2];
        col[i4 + 3] = c4[3];
      }
#pragma unroll
      for (int i = j + 1; i < 16; ++i) t[i] -= col[i] * t[j];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Tm[(16 * w + i) * kLdA + 16 * w + lane] = t[i];
  }
  __syncthreads();
  // off-diagonal blocks by distance d: T_ij = -T_ii * sum_{m=j}^{i-1} A_im T_mj,
  // on fp32 MFMA (16x16x4).  In step s of a 16-deep product lane l supplies
  // k = 4 (l / 16) + s, so its four A values are one float4 of a row, and
  // the B operand of the second product is the first product's accumulator
  // itself (its C layout holds exactly rows 4 (l / 16) + s of column l % 16).
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    const int bi = w + d, bj = w;
    if (bi < 4) {
      f32x4 acc = zero4();
      for (int m = bj; m < bi; ++m) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&Ab[bi * (bi - 1) / 2 + m][r16][4 * grp]);
        const float* tb = &Tm[(16 * m + 4 * grp) * kLdA + 16 * bj + r16];
#pragma unroll
        for (int st = 0; st < 4; ++st) acc = mfma4f32(a4[st], tb[st * kLdA], acc);
      }
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(&Tm[(16 * bi + r16) * kLdA + 16 * bi + 4 * grp]);
      f32x4 res = zero4();
#pragma unroll
      for (int st = 0; st < 4; ++st) res = mfma4f32(d4[st], acc[st], res);
#pragma unroll
      for (int r = 0; r < 4; ++r) Tm[(16 * bi + 4 * grp + r) * kLdA + 16 * bj + r16] = -res[r];
    }
    __syncthreads();
  }

  // Tb = T diag(beta) as fp16 A-operand fragments in the chain's row order:
  // natural row R = 16 w + r16 is row m = 4 ((R / 8) % 4) + R % 4 of rho
  // tile ti = 2 (R / 32) + (R / 4) % 2; lane m + 16 grp of slot tb_slot(ti, b)
  // holds k = 32 b + 8 grp .. + 7
  const int row = 16 * w + r16;
  {
    const int ti = 2 * (w >> 1) + ((r16 >> 2) & 1);
    const int m = 4 * (2 * (w & 1) + (r16 >> 3)) + (r16 & 3);
    u16x8* tdst = ws.tfrag + ((size_t)ci * Hv + h) * 6 * 64 + m + 16 * grp;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (b == 1 && w < 2) break;   // zero block, never read by the chain
      const int c0 = 32 * b + 8 * grp;
      const f32x4 t0v = *reinterpret_cast<const f32x4*>(&Tm[row * kLdA + c0]);
      const f32x4 t1v = *reinterpret_cast<const f32x4*>(&Tm[row * kLdA + c0 + 4]);
      const f32x4 b0v = *reinterpret_cast<const f32x4*>(&Bs[c0]);
      const f32x4 b1v = *reinterpret_cast<const f32x4*>(&Bs[c0 + 4]);
      f32x4 x0, x1;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        x0[ii] = (c0 + ii <= row) ? t0v[ii] * b0v[ii] : 0.f;
        x1[ii] = (c0 + 4 + ii <= row) ? t1v[ii] * b1v[ii] : 0.f;
      }
      tdst[tb_slot(ti, b) * 64] = cat8(f2h4(x0), f2h4(x1));
    }
  }
  if constexpr (BWD) {
    // Tb^T (fp16) and P^T (bf16) A-operand fragments in the reverse chain's
    // rho row order (natural row m = 16 w + r16 as for Tb above): Tb^T[m][kk]
    // = T[kk][m] beta_m (kk >= m) in slot tb_slot(ti, b), P^T[m][kk] =
    // P[kk][m] in slot 2 ti + b; k-block 0 of rho tiles 2 and 3 (natural rows
    // 32..63) is zero in both and never read: not stored
    const int m = 16 * w + r16;
    const float bm = Bs[m];
    const int ti = 2 * (w >> 1) + ((r16 >> 2) & 1);
    const int mr = 4 * (2 * (w & 1) + (r16 >> 3)) + (r16 & 3) + 16 * grp;
    u16x8* ttd = ws.ttfrag + ((size_t)ci * Hv + h) * 6 * 64 + mr;
    u16x8* ptd = ws.ptfrag + (((size_t)ci * Hv + h) * 4 + ti) * 2 * 64 + mr;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (b == 0 && w >= 2) continue;
      f32x4 x0, x1;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int kk = 32 * b + 8 * grp + ii;
        x0[ii] = kk >= m ? Tm[kk * kLdA + m] * bm : 0.f;
        x1[ii] = kk + 4 >= m ? Tm[(kk + 4) * kLdA + m] * bm : 0.f;
      }
      ttd[tb_slot(ti, b) * 64] = cat8(f2h4(x0), f2h4(x1));
      ptd[b * 64] = lds_colfrag(&Ps[0][0], 72, 32 * b, 16 * w, lane);
    }
    // T itself, fp32, its lower blocks only: wave w stores blocks (w, 0..w)
    // of its row tile, one contiguous 1 KB block per store (the diagonal
    // block's upper part is zero in Tm)
    float* tdst = ws.tmat + ((size_t)ci * Hv + h) * kTPacked;
    const int tr = 16 * w + lane / 4, tc4 = 4 * (lane % 4);
    for (int cb = 0; cb <= w; ++cb)
      *reinterpret_cast<f32x4*>(tdst + 256 * tmat_block(w, cb) + 4 * lane) =
          *reinterpret_cast<const f32x4*>(&Tm[tr * kLdA + 16 * cb + tc4]);
  }
}

// ------------------------------------------------------------- host ----
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

WsPlan plan_ws(int B, int T, int Hqk, int Hv, int K, int V, int N, bool has_cu, bool l2,
               bool bwd) {
  WsPlan p{};
  const long long total = (long long)B * T;
  p.ncmax = has_cu ? (total + 63LL * N) / 64 : (long long)B * ((T + 63) / 64);
  const size_t nch = (size_t)p.ncmax * Hv;   // (chunk, v-head) pairs
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t here = at;
    at = align256(at + bytes);
    return here;
  };
  p.off = take((size_t)(N + 1) * 4);
  p.status = take(4);
  p.gate = take(nch * 64 * 4);
  p.tfrag = take(nch * 6 * 64 * 16);
  p.pfrag = take(nch * 6 * 64 * 16);
  // the fp16 K / Q copies, where the chains do not read the caller's rows:
  // Q only with use_qk_l2norm (normalised), K also for the backward and for
  // two V tiles per workgroup
  const size_t nqk = (size_t)p.ncmax * Hqk;   // (chunk, qk-head) pairs
  p.k16_copy = !chain_reads_rows(bwd, l2, N, Hv, V);
  p.q16_copy = l2;
  p.k16 = take(p.k16_copy ? nqk * (K == 128 ? KLayout<128>::BYTES : KLayout<64>::BYTES) : 0);
  p.q16 = take(p.q16_copy ? nqk * 64 * K * 2 : 0);
  p.qn = p.kn = at;
  if (l2 && bwd) {
    p.qn = take((size_t)total * Hqk * K * 2);
    p.kn = take((size_t)total * Hqk * K * 2);
  }
  if (bwd) {
    p.tmat = take(nch * kTPacked * 4);
    p.ttfrag = take(nch * 6 * 64 * 16);
    p.ptfrag = take(nch * 4 * 2 * 64 * 16);
    p.hs = take(nch * K * V * 2);
    p.dse = take(nch * K * V * 2);
    p.dl = take(nch * 64 * V * 2);
    p.dd = take(nch * 64 * V * 2);
    p.qtfrag = take((size_t)p.ncmax * Hqk * (K / 16) * 2 * 64 * 16);
  }
  p.total = at;
  return p;
}

ChunkWs ws_pointers(const WsPlan& p, unsigned char* wsb) {
  ChunkWs ws{};
  ws.off = reinterpret_cast<int32_t*>(wsb + p.off);
  ws.status = reinterpret_cast<int32_t*>(wsb + p.status);
  ws.gate = reinterpret_cast<float*>(wsb + p.gate);
  ws.tfrag = reinterpret_cast<u16x8*>(wsb + p.tfrag);
  ws.pfrag = reinterpret_cast<u16x8*>(wsb + p.pfrag);
  ws.k16 = p.k16_copy ? wsb + p.k16 : nullptr;
  ws.q16 = p.q16_copy ? reinterpret_cast<u16x8*>(wsb + p.q16) : nullptr;
  ws.qn = reinterpret_cast<uint16_t*>(wsb + p.qn);
  ws.kn = reinterpret_cast<uint16_t*>(wsb + p.kn);
  if (p.hs) {
    ws.tmat = reinterpret_cast<float*>(wsb + p.tmat);
    ws.ttfrag = reinterpret_cast<u16x8*>(wsb + p.ttfrag);
    ws.ptfrag = reinterpret_cast<u16x8*>(wsb + p.ptfrag);
    ws.qtfrag = reinterpret_cast<u16x8*>(wsb + p.qtfrag);
    ws.hs = reinterpret_cast<uint16_t*>(wsb + p.hs);
    ws.dl = reinterpret_cast<uint16_t*>(wsb + p.dl);
  }
  return ws;
}

template <int K, bool BWD, bool OUT>
static void launch_chunk(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const float* g, const float* beta, const float* h0, float* ht,
                         uint16_t* o, const int32_t* cu, int B, int T, int Hqk, int Hv, int V,
                         int N, float scale, bool l2, const WsPlan& p, unsigned char* wsb,
                         hipStream_t st, const GateIn& gate) {
  const ChunkWs ws = ws_pointers(p, wsb);
  const int total = B * T;
  if (cu)
    hipLaunchKernelGGL(chunk_table_kernel, dim3(1), dim3(256), 0, st, cu, N, T, total,
                       (int)p.ncmax, ws.off, ws.status);
  if (p.ncmax > 0) {
    if (l2)
      hipLaunchKernelGGL((chunk_prep_kernel<K, BWD, OUT, true>), dim3((unsigned)p.ncmax, Hv), dim3(256),
                         0, st, q, k, g, beta, cu, N, T, total, Hqk, Hv, scale, ws, gate);
    else
      hipLaunchKernelGGL((chunk_prep_kernel<K, BWD, OUT, false>), dim3((unsigned)p.ncmax, Hv), dim3(256),
                         0, st, q, k, g, beta, cu, N, T, total, Hqk, Hv, scale, ws, gate);
  }
  // the chain reads K and Q as the prep kernel's fp16 copies where the plan
  // has them (normalised with use_qk_l2norm), else as the caller's bf16 rows
  launch_chain_sw<K, BWD, OUT>(v, ws.q16 ? nullptr : q, ws.k16 ? nullptr : k, h0,
                               OUT ? ht : nullptr, OUT ? o : nullptr, cu, N, T, total, Hqk, Hv,
                               V, scale, ws, st);
  // a cu_seqlens violation left every sequence empty: o is zero-filled (and
  // ht = h0, written by the chain for an empty sequence)
  if (cu && OUT) {
    ZeroList z{};
    z.p[0] = o;
    z.bytes[0] = (size_t)total * Hv * V * 2;
    launch_zero_on_violation(ws.status, z, st);
  }
}

void launch_chunk_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                      const float* beta, const float* h0, float* ht, uint16_t* o,
                      const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N,
                      float scale, bool l2, FwdMode mode, const WsPlan& p, unsigned char* wsb,
                      hipStream_t st, const GateIn& gate) {
#define GDN_FWD(KK_, BWD_, OUT_)                                                             \
  launch_chunk<KK_, BWD_, OUT_>(q, k, v, g, beta, h0, ht, o, cu, B, T, Hqk, Hv, V, N, scale, l2, \
                                p, wsb, st, gate)
  if (K == 128) {
    if (mode == FwdMode::kForward) GDN_FWD(128, false, true);
    else if (mode == FwdMode::kRecompute) GDN_FWD(128, true, false);
    else GDN_FWD(128, true, true);
  } else {
    if (mode == FwdMode::kForward) GDN_FWD(64, false, true);
    else if (mode == FwdMode::kRecompute) GDN_FWD(64, true, false);
    else GDN_FWD(64, true, true);
  }
#undef GDN_FWD
}

}  // namespace gdn

namespace gdn_host {
int validate_gate(const char* name, const void* A_log, const void* dt_bias, int a_dtype,
                  int b_dtype, int p_dtype, float sp_beta, long long tokens);
int validate_gate_size(const char* name, long long elements);
int validate_common(const void* q, const void* k, const void* v, const float* g,
                    const float* beta, const float* h0, const float* ht, const void* o,
                    const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N);
}

extern "C" size_t gdn_chunk_workspace_bytes(int B, int T, int Hqk, int Hv, int K, int V,
                                            int N, int has_cu_seqlens, int use_qk_l2norm) {
  if (B < 0 || T < 0 || Hqk <= 0 || Hv <= 0 || N < 0 || K <= 0 || V <= 0) return 0;
  return gdn::plan_ws(B, T, Hqk, Hv, K, V, N, has_cu_seqlens != 0, use_qk_l2norm != 0, false)
      .total;
}

namespace {
int chunk_fwd_impl(const void* q, const void* k, const void* v, const float* g,
                   const float* beta, const float* h0, float* ht, void* o,
                   const int32_t* cu_seqlens, int B, int T, int Hqk, int Hv, int K, int V, int N,
                   float scale, int use_qk_l2norm, void* workspace, size_t workspace_bytes,
                   const gdn::GateIn& gate, void* stream, const char* name) {
  if (N == 0 || ((long long)B * T == 0 && !ht)) return GDN_OK;  // nothing to compute
  gdn_host::launch_begin();
  const gdn::WsPlan p = gdn::plan_ws(B, T, Hqk, Hv, K, V, N, cu_seqlens != nullptr,
                                     use_qk_l2norm != 0, false);
  if (!workspace || workspace_bytes < p.total)
    return gdn_host::fail(GDN_ERR_WORKSPACE, std::string(name) + ": workspace needs " +
                                                 std::to_string(p.total) + " bytes, got " +
                                                 std::to_string(workspace_bytes));
  if (p.ncmax > (1LL << 30) || (long long)N * Hv * (V / 16) >= (1LL << 31))
    return gdn_host::fail(GDN_ERR_SHAPE, std::string(name) + ": problem too large");
  gdn::launch_chunk_fwd(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                        static_cast<const uint16_t*>(v), g, beta, h0, ht,
                        static_cast<uint16_t*>(o), cu_seqlens, B, T, Hqk, Hv, K, V, N, scale,
                        use_qk_l2norm != 0, gdn::FwdMode::kForward, p,
                        static_cast<unsigned char*>(workspace), static_cast<hipStream_t>(stream),
                        gate);
  return gdn_host::check_launch(name);
}
}  // namespace

extern "C" int gdn_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                             const float* beta, const float* h0, float* ht, void* o,
                             const int32_t* cu_seqlens, int B, int T, int Hqk, int Hv, int K,
                             int V, int N, float scale, int use_qk_l2norm, void* workspace,
                             size_t workspace_bytes, void* stream) {
  const int rc = gdn_host::validate_common(q, k, v, g, beta, h0, ht, o, cu_seqlens, B, T, Hqk,
                                           Hv, K, V, N);
  if (rc) return rc;
  return chunk_fwd_impl(q, k, v, g, beta, h0, ht, o, cu_seqlens, B, T, Hqk, Hv, K, V, N, scale,
                        use_qk_l2norm, workspace, workspace_bytes, gdn::GateIn{}, stream,
                        "gdn_chunk_fwd");
}

// Prefill with the gating computed inside (declared in gdn_layer.h): the prep
// kernel forms g and beta from (A_log, a, b, dt_bias); no g / beta tensor.
extern "C" int gdn_chunk_fwd_gating(const void* q, const void* k, const void* v,
                                    const void* A_log, const void* a, const void* b,
                                    const void* dt_bias, int a_dtype, int b_dtype, int p_dtype,
                                    float sp_beta, float sp_threshold, const float* h0,
                                    float* ht, void* o, const int32_t* cu_seqlens, int B, int T,
                                    int Hqk, int Hv, int K, int V, int N, float scale,
                                    int use_qk_l2norm, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  const char* name = "gdn_chunk_fwd_gating";
  int rc = gdn_host::validate_common(q, k, v, static_cast<const float*>(a),
                                     static_cast<const float*>(b), h0, ht, o, cu_seqlens, B, T,
                                     Hqk, Hv, K, V, N);
  if (rc) return rc;
  rc = gdn_host::validate_gate(name, A_log, dt_bias, a_dtype, b_dtype, p_dtype, sp_beta,
                               (long long)B * T);
  if (rc) return rc;
  rc = gdn_host::validate_gate_size(name, (long long)B * T * Hv);
  if (rc) return rc;
  const gdn::GateIn gate{A_log, a, b, dt_bias, a_dtype, b_dtype, p_dtype, sp_beta, sp_threshold,
                         (long long)B * T * Hv, Hv};
  return chunk_fwd_impl(q, k, v, nullptr, nullptr, h0, ht, o, cu_seqlens, B, T, Hqk, Hv, K, V, N,
                        scale, use_qk_l2norm, workspace, workspace_bytes, gate, stream, name);
}

// ----------------------------------------------- allocation-free form ----
// Device scratch of gdn_chunk_fwd_noalloc: one array per GPU the library runs
// on, held until the process ends.  Its name is a host-side stand-in: host
// code uses the per-device address from hipGetSymbolAddress, never the name.
constexpr size_t kNoAllocScratchBytes = GDN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
using gdn::kMaxDevices;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];   // address of `scratch` on each device, once looked up

// Address of the current device's scratch (looked up once per device).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return gdn_host::fail(static_cast<int>(e), std::string("gdn_chunk_fwd_noalloc: hipGetDevice: ") +
                                                   hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_chunk_fwd_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    // relaxed capture mode for this thread, so that a first call made under
    // stream capture may look the symbol up (it enqueues nothing)
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t me = hipThreadExchangeStreamCaptureMode(&mode);
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (me == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || !ptr)
      return gdn_host::fail(e != hipSuccess ? static_cast<int>(e) : GDN_ERR_NULL,
                            std::string("gdn_chunk_fwd_noalloc: hipGetSymbolAddress: ") +
                                hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GDN_OK;
}
}  // namespace

// gdn_chunk_fwd with the library's own scratch in place of a workspace
// (declared in gdn.h): no allocation of any kind.
extern "C" int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const float* g,
                                     const float* beta, const float* h0, float* ht, void* o,
                                     const int32_t* cu_seqlens, int B, int T, int Hqk, int Hv,
                                     int K, int V, int N, float scale, int use_qk_l2norm,
                                     void* stream) {
  int rc = gdn_host::validate_common(q, k, v, g, beta, h0, ht, o, cu_seqlens, B, T, Hqk, Hv,
                                     K, V, N);
  if (rc) return rc;
  if (N == 0 || ((long long)B * T == 0 && !ht)) return GDN_OK;  // nothing to compute
  gdn_host::launch_begin();
  const gdn::WsPlan p = gdn::plan_ws(B, T, Hqk, Hv, K, V, N, cu_seqlens != nullptr,
                                     use_qk_l2norm != 0, false);
  if (p.total > kNoAllocScratchBytes)
    return gdn_host::fail(GDN_ERR_WORKSPACE,
                          "gdn_chunk_fwd_noalloc: the problem needs " + std::to_string(p.total) +
                              " bytes of scratch, more than the library's " +
                              std::to_string(kNoAllocScratchBytes) +
                              " (use gdn_chunk_fwd with a workspace)");
  if (p.ncmax > (1LL << 30) || (long long)N * Hv * (V / 16) >= (1LL << 31))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_chunk_fwd_noalloc: problem too large");
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  gdn::launch_chunk_fwd(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                        static_cast<const uint16_t*>(v), g, beta, h0, ht,
                        static_cast<uint16_t*>(o), cu_seqlens, B, T, Hqk, Hv, K, V, N, scale,
                        use_qk_l2norm != 0, gdn::FwdMode::kForward, p,
                        static_cast<unsigned char*>(ws), static_cast<hipStream_t>(stream));
  return gdn_host::check_launch("gdn_chunk_fwd_noalloc");
}

extern "C" int gdn_chunk_fwd_save(const void* q, const void* k, const void* v, const float* g,
                                  const float* beta, const float* h0, float* ht, void* o,
                                  const int32_t* cu_seqlens, int B, int T, int Hqk, int Hv, int K,
                                  int V, int N, float scale, int use_qk_l2norm, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  int rc = gdn_host::validate_common(q, k, v, g, beta, h0, ht, o, cu_seqlens, B, T, Hqk, Hv,
                                     K, V, N);
  if (rc) return rc;
  if (N == 0 || ((long long)B * T == 0 && !ht)) return GDN_OK;  // nothing to compute
  gdn_host::launch_begin();
  const gdn::WsPlan p = gdn::plan_ws(B, T, Hqk, Hv, K, V, N, cu_seqlens != nullptr,
                                     use_qk_l2norm != 0, true);
  if (!workspace || workspace_bytes < p.total)
    return gdn_host::fail(GDN_ERR_WORKSPACE, "gdn_chunk_fwd_save: workspace needs " +
                                                 std::to_string(p.total) + " bytes, got " +
                                                 std::to_string(workspace_bytes));
  if (p.ncmax > (1LL << 30) || (long long)N * Hv * (V / 16) >= (1LL << 31))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_chunk_fwd_save: problem too large");
  gdn::launch_chunk_fwd(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                        static_cast<const uint16_t*>(v), g, beta, h0, ht,
                        static_cast<uint16_t*>(o), cu_seqlens, B, T, Hqk, Hv, K, V, N, scale,
                        use_qk_l2norm != 0, gdn::FwdMode::kSave, p,
                        static_cast<unsigned char*>(workspace), static_cast<hipStream_t>(stream));
  return gdn_host::check_launch("gdn_chunk_fwd_save");
}
