// Fused recurrent gated delta rule for gfx950 (decode: one token per
// sequence; also multi-token / varlen).
//
// Operator semantics: transformers modeling_qwen3_next.py:490-501 (the
// token loop of torch_recurrent_gated_delta_rule); the reference repository
// has no GDN code, its launcher convention is backends/amdgpu/driver.py:
// 324-343 (raw pointers + scalars + caller stream).
//
// Design: the path is HBM-bound (0.8 flop/B), so there is no MFMA.  A
// workgroup of NT lanes advances one (sequence, v-head) state tile S[K][V]
// at a time (fp32, 64 KiB at K = V = 128, where NT = 512: measured on
// MI355X, 512 lanes x 8 float4 per 64 KiB tile streams an in-place
// read-modify-write faster than 256 lanes x 16), and a persistent grid of
// 1024 workgroups (4 per CU) walks the tiles with the next tile's state
// loaded while the current one is advanced: 6.27 TB/s at batch 256 against
// 5.35 TB/s for one workgroup per tile.  Each lane holds a
// float4 column group of K/ROWG rows in VGPRs; the tile is read once with
// coalesced 16-byte nontemporal loads (a wavefront covers whole contiguous
// rows), advanced through every token of the sequence in registers, and
// written once.  Per token, the two reductions over K (S^T k and S^T q) and
// the scalars k.q, |k|^2, |q|^2 come from one pass over the registers: lane
// partials, a xor-shuffle across the row groups inside a wavefront, then an
// NT/64-way LDS combine.
// Using the pre-update S,
//     S' = e^g S + k (x) d,   d = beta (v - e^g S^T k),
//     o  = scale (e^g S^T q + d (k.q))
// so the updated tile never has to be re-read.
#include "gdn_common.h"

namespace gdn {

// Cache-policy bits of a raw buffer access on gfx950: NT (streaming).
constexpr int kNonTemporal = 2;
#ifndef GDN_DECODE_GRID
#define GDN_DECODE_GRID 1024
#endif
// workgroups of the persistent decode grid
constexpr int kDecodeGrid = GDN_DECODE_GRID;
// pool slots and sequences up to which the shared-slot check of a slot
// table runs once per workgroup in LDS (beyond: at every tile)
constexpr int kSlotOwn = 4096;
constexpr int kSlotSeq = 4096;

// Persistent form: a workgroup walks tiles blockIdx.x, +G, +2G, ... and
// loads the next tile's state while it advances the current one, so the
// state stream never waits for the per-token reductions.  State loads go
// through a buffer resource whose size is 0 for a tile that has nothing to
// load (past the end, padding slot, no h0): those loads return zeros and
// touch no memory, so the prefetch needs no branch.
// GATE: g and beta formed in the kernel from `gate`; otherwise read from g /
// beta.
template <int K, int V, int NT, bool GATE>
__global__ __launch_bounds__(NT) void recurrent_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ beta, const float* h0, float* ht,
    uint16_t* __restrict__ o, const int32_t* __restrict__ cu, int T,
    int total_tokens, int Hqk, int Hv, float scale, int l2norm,
    const int32_t* __restrict__ slots, int num_slots, int ntiles, int slot_stride,
    const int32_t* __restrict__ accepted, GateIn gate) {
  constexpr int COLG = V / 4;          // float4 column groups per row
  constexpr int ROWG = NT / COLG;      // row groups
  constexpr int RPT = K / ROWG;        // rows per lane
  constexpr int NW = NT / 64;          // wavefronts
  constexpr int NRED = 11;             // kv[4], sq[4], kq, kk, qq
  static_assert(ROWG * COLG == NT && RPT * ROWG == K, "tile shape");
  static_assert(COLG <= 64 && 64 % COLG == 0, "wave covers whole rows");

  __shared__ float kq_s[2][K];
  __shared__ float red[NW][COLG][NRED + 1];
  __shared__ float gsh[2];   // GATE: g, beta of a tile's first token
  __shared__ int sown[kSlotOwn];              // slot tables: lowest sequence per slot
  __shared__ unsigned sflag[kSlotSeq / 32];   // and a bit per sequence sharing one

  const int tid = threadIdx.x;
  const int cg = tid % COLG;
  const int rg = tid / COLG;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int G = gridDim.x;

  // state slot a tile (sequence n, v-head h) starts from; under continuous
  // batching a slot outside the pool marks a padding sequence, left
  // untouched.  Speculative decoding (slot_stride > 0): the slots of sequence
  // n are row n of a [N][slot_stride] table, the state after token t goes to
  // entry t, and the initial state is entry accepted[n] - 1 (entry 0 without
  // `accepted`), the state after the last accepted token of the previous step.
  auto slot_of = [&](int tile) {
    const int n = tile / Hv;
    int slot = n;
    if (slots) {
      int col = 0;
      if (slot_stride > 0 && accepted) {
        col = accepted[n] - 1;
        if (col < 0 || col >= slot_stride) return -1;
      }
      slot = slots[(size_t)n * (slot_stride > 0 ? slot_stride : 1) + col];
      if (slot < 0 || slot >= num_slots) slot = -1;
    }
    return slot;
  };
  // GATE: the tile's first-token gate inputs are loaded with its state (and
  // ahead of it), one tile before they are used
  auto load_state = [&](f32x4 (&S)[RPT], GateRaw& gr, int tile) {
    const int tl = min(tile, ntiles - 1);
    if constexpr (GATE) {
      const int n = tl / Hv;
      const int s = cu ? min(max(cu[n], 0), total_tokens) : n * T;
      gr = gate_load(gate, (long long)s * Hv + tl % Hv, tl % Hv);
    }
    const int slot = slot_of(tl);
    const bool live = h0 && tile < ntiles && slot >= 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(h0) + (live ? ((size_t)slot * Hv + tl % Hv) * (size_t)K * V : 0), 0,
        live ? K * V * 4 : 0, kBufferFlags);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      S[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
          rs, ((rg + ROWG * i) * COLG + cg) * 16, 0, kNonTemporal));
  };

  // Shared slots, checked on the device: the slot value of entry j of table
  // row m if sequence m reads or writes it, else -1 (continuous batching:
  // the row's one entry; speculative decoding: the initial entry and the
  // entries of the tokens it has, none for a padding sequence)
  const int srow = slot_stride > 0 ? slot_stride : 1;
  auto touched = [&](int m, int j) -> int {
    const int x = slots[(size_t)m * srow + j];
    if (x < 0 || x >= num_slots) return -1;
    if (slot_stride == 0) return x;
    int col = 0;
    if (accepted) {
      col = accepted[m] - 1;
      if (col < 0 || col >= slot_stride) return -1;
    }
    const int init = slots[(size_t)m * slot_stride + col];
    if (init < 0 || init >= num_slots) return -1;
    if (j == col) return x;
    int len = T;
    if (cu) {
      const int a = min(max(cu[m], 0), total_tokens);
      len = min(max(cu[m + 1], a), total_tokens) - a;
    }
    return j < len ? x : -1;
  };
  // Which sequences share a slot does not depend on the tile, so with at
  // most kSlotOwn slots and kSlotSeq sequences a workgroup finds them all
  // once, before its first tile: the lowest sequence touching each slot
  // (LDS atomic min), then every entry whose slot has another lowest
  // sequence marks both sequences (a bit per sequence).  A tile then reads
  // its sequence's bit.  Larger tables are scanned at every tile instead.
  const int nseq = ntiles / Hv;
  const int nent = slots ? nseq * srow : 0;
  const bool own_lds = num_slots <= kSlotOwn && nseq <= kSlotSeq;
  if (slots && own_lds) {
    for (int x = tid; x < num_slots; x += NT) sown[x] = 0x7fffffff;
    for (int w = tid; w < (nseq + 31) / 32; w += NT) sflag[w] = 0u;
    __syncthreads();
    for (int idx = tid; idx < nent; idx += NT) {
      const int x = touched(idx / srow, idx % srow);
      if (x >= 0) atomicMin(&sown[x], idx / srow);
    }
    __syncthreads();
    for (int idx = tid; idx < nent; idx += NT) {
      const int m = idx / srow;
      const int x = touched(m, idx % srow);
      if (x < 0) continue;
      const int first = sown[x];
      if (first != m) {
        atomicOr(&sflag[m >> 5], 1u << (m & 31));
        atomicOr(&sflag[first >> 5], 1u << (first & 31));
      }
    }
    __syncthreads();
  }
  // whether a slot sequence n touches is also touched by another sequence
  // (same answer in every thread of the workgroup)
  auto shares_slot = [&](int n) -> bool {
    if (own_lds) return (sflag[n >> 5] >> (n & 31)) & 1u;
    bool hit = false;
    for (int idx = tid; idx < nent; idx += NT) {
      if (idx / srow == n) continue;
      const int x = touched(idx / srow, idx % srow);
      if (x < 0) continue;
      for (int j = 0; j < srow; ++j) hit |= touched(n, j) == x;
    }
    return __syncthreads_or(hit) != 0;
  };

  auto run_tile = [&](f32x4 (&S)[RPT], const GateRaw& gr, int tile) {
    const int slot = slot_of(tile);
    if (slot < 0) return;
    const int h = tile % Hv;
    const int n = tile / Hv;
    const int hq = h / (Hv / Hqk);
    int s, e;
    if (cu) {
      s = min(max(cu[n], 0), total_tokens);
      e = min(max(cu[n + 1], s), total_tokens);
    } else {
      s = n * T;
      e = s + T;
    }
    if (slots && shares_slot(n)) {
      // a slot two sequences would use: neither advances it (no state is
      // written, so the pool is never written concurrently) and its output
      // rows are NaN, so the caller's error shows
      if (rg == 0) {
        const u16x4 nan4 = {0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0};
        for (int t = s; t < e; ++t)
          *reinterpret_cast<u16x4*>(o + ((size_t)t * Hv + h) * V + 4 * cg) = nan4;
      }
      return;
    }
    for (int t = s; t < e; ++t) {
      if (GATE && t == s && wave == NW - 1) {
        // the first token's gate, from inputs loaded a tile ahead: formed
        // by the one wave that stages no k / q row, before the loads whose
        // wait would also cover the next tile's state prefetch, so the math
        // overlaps that prefetch; shared through LDS at the barrier below
        float g0, b0;
        gate_eval(gate, gr, g0, b0);
        if (lane == 0) {
          gsh[0] = g0;
          gsh[1] = b0;
        }
      }
      const size_t qk_row = ((size_t)t * Hqk + hq) * K;
      // speculative decoding: slot receiving the state after this token
      int tslot = -1;
      if (slot_stride > 0 && t - s < slot_stride) {
        tslot = slots[(size_t)n * slot_stride + (t - s)];
        if (tslot >= num_slots) tslot = -1;
      }
      if (tid < K) {
        kq_s[0][tid] = bf2f(k[qk_row + tid]);
        kq_s[1][tid] = bf2f(q[qk_row + tid]);
      }
      const size_t vh = (size_t)t * Hv + h;
      const u16x4 vb = *reinterpret_cast<const u16x4*>(v + vh * V + 4 * cg);
      float gt = 0.f, bt = 0.f;
      if constexpr (GATE) {
        // later tokens (multi-token steps): formed here
        if (t > s) {
          float neg_a, dtb;
          gate_head<true>(gate, h, neg_a, dtb);
          gate_elem<true>(gate, (long long)vh, neg_a, dtb, gt, bt);
        }
      } else {
        gt = g[vh];
        bt = beta[vh];
      }
      __syncthreads();
      if (GATE && t == s) {
        gt = gsh[0];
        bt = gsh[1];
      }

      float r[NRED];
      float kreg[RPT];  // k rows kept in VGPRs: kq_s is restaged by the next token
#pragma unroll
      for (int j = 0; j < NRED; ++j) r[j] = 0.f;
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float kr = kq_s[0][rg + ROWG * i];
        const float qr = kq_s[1][rg + ROWG * i];
        kreg[i] = kr;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          r[c] += S[i][c] * kr;
          r[4 + c] += S[i][c] * qr;
        }
        r[8] += kr * qr;
        r[9] += kr * kr;
        r[10] += qr * qr;
      }
#pragma unroll
      for (int off = COLG; off < 64; off *= 2) {
#pragma unroll
        for (int j = 0; j < NRED; ++j) r[j] += __shfl_xor(r[j], off);
      }
      if (lane < COLG) {
#pragma unroll
        for (int j = 0; j < NRED; ++j) red[wave][cg][j] = r[j];
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NRED; ++j) {
        float acc = red[0][cg][j];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) acc += red[ww][cg][j];
        r[j] = acc;
      }

      const float ik = l2norm ? rsqrtf(r[9] + 1e-6f) : 1.f;
      const float iq = l2norm ? rsqrtf(r[10] + 1e-6f) : 1.f;
      const float eg = __expf(gt);
      float d[4];
      float ov[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        d[c] = bt * (bf2f(vb[c]) - eg * r[c] * ik);
        ov[c] = scale * iq * (eg * r[4 + c] + d[c] * r[8] * ik);
      }
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float kr = kreg[i] * ik;
#pragma unroll
        for (int c = 0; c < 4; ++c) S[i][c] = eg * S[i][c] + kr * d[c];
      }
      if (rg == 0) {
        u16x4 ob;
#pragma unroll
        for (int c = 0; c < 4; ++c) ob[c] = f2bf(ov[c]);
        *reinterpret_cast<u16x4*>(o + vh * V + 4 * cg) = ob;
      }
      if (ht && tslot >= 0) {
        f32x4* dst = reinterpret_cast<f32x4*>(ht + ((size_t)tslot * Hv + h) * (size_t)K * V);
#pragma unroll
        for (int i = 0; i < RPT; ++i)
          __builtin_nontemporal_store(S[i], dst + (size_t)(rg + ROWG * i) * COLG + cg);
      }
    }
    if (ht && slot_stride == 0) {
      f32x4* dst = reinterpret_cast<f32x4*>(ht + ((size_t)slot * Hv + h) * (size_t)K * V);
#pragma unroll
      for (int i = 0; i < RPT; ++i)
        __builtin_nontemporal_store(S[i], dst + (size_t)(rg + ROWG * i) * COLG + cg);
    }
  };

  int t = blockIdx.x;
  if (t >= ntiles) return;
  f32x4 SA[RPT], SB[RPT];
  GateRaw gA{}, gB{};
  load_state(SA, gA, t);
  for (;;) {
    load_state(SB, gB, t + G);
    run_tile(SA, gA, t);
    t += G;
    if (t >= ntiles) break;
    load_state(SA, gA, t + G);
    run_tile(SB, gB, t);
    t += G;
    if (t >= ntiles) break;
  }
}

template <int K, int V>
static void launch_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             const float* g, const float* beta, const float* h0,
                             float* ht, uint16_t* o, const int32_t* cu, int B, int T,
                             int Hqk, int Hv, int N, float scale, int l2norm,
                             const int32_t* slots, int num_slots, hipStream_t stream,
                             int slot_stride = 0, const int32_t* accepted = nullptr,
                             const GateIn& gate = GateIn{}) {
  const int total_tokens = B * T;
  constexpr int NT = (K * V >= 128 * 128) ? 512 : 256;
  const int ntiles = N * Hv;
  // persistent workgroups: enough to fill every CU several times over, each
  // walking ntiles / grid tiles with the next state prefetched
  const int grid = ntiles < kDecodeGrid ? ntiles : kDecodeGrid;
  if (gate.a)
    hipLaunchKernelGGL((recurrent_kernel<K, V, NT, true>), dim3(grid), dim3(NT), 0, stream, q,
                       k, v, g, beta, h0, ht, o, cu, T, total_tokens, Hqk, Hv, scale, l2norm,
                       slots, num_slots, ntiles, slot_stride, accepted, gate);
  else
    hipLaunchKernelGGL((recurrent_kernel<K, V, NT, false>), dim3(grid), dim3(NT), 0, stream, q,
                       k, v, g, beta, h0, ht, o, cu, T, total_tokens, Hqk, Hv, scale, l2norm,
                       slots, num_slots, ntiles, slot_stride, accepted, gate);
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

namespace {
// gdn_recurrent_fwd and its gating form
int recurrent_plain(const void* q, const void* k, const void* v, const float* g,
                    const float* beta, const float* h0, float* ht, void* o,
                    const int32_t* cu_seqlens, int B, int T, int Hqk, int Hv, int K, int V, int N,
                    float scale, int use_qk_l2norm, const gdn::GateIn& gate, void* stream,
                    const char* name) {
  if (N == 0 || ((long long)B * T == 0 && !ht)) return GDN_OK;  // nothing to compute
  gdn_host::launch_begin();
  auto* qq = static_cast<const uint16_t*>(q);
  auto* kk = static_cast<const uint16_t*>(k);
  auto* vv = static_cast<const uint16_t*>(v);
  auto* oo = static_cast<uint16_t*>(o);
  auto st = static_cast<hipStream_t>(stream);
#define GDN_REC(KK, VV)                                                                   \
  if (K == KK && V == VV) {                                                               \
    gdn::launch_recurrent<KK, VV>(qq, kk, vv, g, beta, h0, ht, oo, cu_seqlens, B, T, Hqk, \
                                  Hv, N, scale, use_qk_l2norm, nullptr, N, st, 0, nullptr, \
                                  gate);                                                  \
    return gdn_host::check_launch(name);                                                  \
  }
  GDN_REC(128, 128)
  GDN_REC(64, 64)
  GDN_REC(128, 64)
  GDN_REC(64, 128)
#undef GDN_REC
  return gdn_host::fail(GDN_ERR_SHAPE, std::string(name) + ": unsupported K/V");
}

// gdn_recurrent_fwd_indexed and the gating form with state indices
int recurrent_indexed(const void* q, const void* k, const void* v, const float* g,
                      const float* beta, const float* h0, float* ht, void* o,
                      const int32_t* cu_seqlens, const int32_t* state_indices, int B, int T,
                      int Hqk, int Hv, int K, int V, int N, int num_slots, float scale,
                      int use_qk_l2norm, const gdn::GateIn& gate, void* stream,
                      const char* name) {
  if (num_slots < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, std::string(name) + ": num_slots must be >= 0");
  if (N > 0 && !state_indices)
    return gdn_host::fail(GDN_ERR_NULL, std::string(name) + ": state_indices must be non-NULL");
  if (ht && h0 && ht != h0) {
    const size_t sb = (size_t)num_slots * Hv * K * V * sizeof(float);
    const auto pa = reinterpret_cast<uintptr_t>(h0), pb = reinterpret_cast<uintptr_t>(ht);
    if (pa < pb + sb && pb < pa + sb)
      return gdn_host::fail(GDN_ERR_ALIAS, std::string(name) + ": ht must equal h0 exactly or not overlap it");
  }
  if (N == 0 || num_slots == 0 || ((long long)B * T == 0 && !ht)) return GDN_OK;
  gdn_host::launch_begin();
  auto* qq = static_cast<const uint16_t*>(q);
  auto* kk = static_cast<const uint16_t*>(k);
  auto* vv = static_cast<const uint16_t*>(v);
  auto* oo = static_cast<uint16_t*>(o);
  auto st = static_cast<hipStream_t>(stream);
#define GDN_RECI(KK, VV)                                                                  \
  if (K == KK && V == VV) {                                                               \
    gdn::launch_recurrent<KK, VV>(qq, kk, vv, g, beta, h0, ht, oo, cu_seqlens, B, T, Hqk, \
                                  Hv, N, scale, use_qk_l2norm, state_indices, num_slots,  \
                                  st, 0, nullptr, gate);                                  \
    return gdn_host::check_launch(name);                                                  \
  }
  GDN_RECI(128, 128)
  GDN_RECI(64, 64)
  GDN_RECI(128, 64)
  GDN_RECI(64, 128)
#undef GDN_RECI
  return gdn_host::fail(GDN_ERR_SHAPE, std::string(name) + ": unsupported K/V");
}
}  // namespace

extern "C" int gdn_recurrent_fwd(const void* q, const void* k, const void* v,
                                 const float* g, const float* beta, const float* h0,
                                 float* ht, void* o, const int32_t* cu_seqlens, int B,
                                 int T, int Hqk, int Hv, int K, int V, int N, float scale,
                                 int use_qk_l2norm, void* stream) {
  const int rc = gdn_host::validate_common(q, k, v, g, beta, h0, ht, o, cu_seqlens, B, T, Hqk,
                                           Hv, K, V, N);
  if (rc) return rc;
  return recurrent_plain(q, k, v, g, beta, h0, ht, o, cu_seqlens, B, T, Hqk, Hv, K, V, N, scale,
                         use_qk_l2norm, gdn::GateIn{}, stream, "gdn_recurrent_fwd");
}

// Continuous batching: sequence n advances state slot state_indices[n] of a
// [num_slots, Hv, K, V] pool (declared in gdn_layer.h).
extern "C" int gdn_recurrent_fwd_indexed(const void* q, const void* k, const void* v,
                                         const float* g, const float* beta, const float* h0,
                                         float* ht, void* o, const int32_t* cu_seqlens,
                                         const int32_t* state_indices, int B, int T, int Hqk,
                                         int Hv, int K, int V, int N, int num_slots,
                                         float scale, int use_qk_l2norm, void* stream) {
  const int rc = gdn_host::validate_common(q, k, v, g, beta, nullptr, nullptr, o, cu_seqlens,
                                           B, T, Hqk, Hv, K, V, N);
  if (rc) return rc;
  return recurrent_indexed(q, k, v, g, beta, h0, ht, o, cu_seqlens, state_indices, B, T, Hqk,
                           Hv, K, V, N, num_slots, scale, use_qk_l2norm, gdn::GateIn{}, stream,
                           "gdn_recurrent_fwd_indexed");
}

// Decode with the gating computed inside (declared in gdn_layer.h): g and
// beta come from (A_log, a, b, dt_bias) in the kernel, not from HBM.
extern "C" int gdn_recurrent_fwd_gating(const void* q, const void* k, const void* v,
                                        const void* A_log, const void* a, const void* b,
                                        const void* dt_bias, int a_dtype, int b_dtype,
                                        int p_dtype, float sp_beta, float sp_threshold,
                                        const float* h0, float* ht, void* o,
                                        const int32_t* cu_seqlens, const int32_t* state_indices,
                                        int B, int T, int Hqk, int Hv, int K, int V, int N,
                                        int num_slots, float scale, int use_qk_l2norm,
                                        void* stream) {
  const char* name = "gdn_recurrent_fwd_gating";
  int rc = gdn_host::validate_common(q, k, v, static_cast<const float*>(a),
                                     static_cast<const float*>(b), state_indices ? nullptr : h0,
                                     state_indices ? nullptr : ht, o, cu_seqlens, B, T, Hqk, Hv,
                                     K, V, N);
  if (rc) return rc;
  rc = gdn_host::validate_gate(name, A_log, dt_bias, a_dtype, b_dtype, p_dtype, sp_beta,
                               (long long)B * T);
  if (rc) return rc;
  rc = gdn_host::validate_gate_size(name, (long long)B * T * Hv);
  if (rc) return rc;
  const gdn::GateIn gate{A_log, a, b, dt_bias, a_dtype, b_dtype, p_dtype, sp_beta, sp_threshold,
                         (long long)B * T * Hv, Hv};
  if (state_indices)
    return recurrent_indexed(q, k, v, nullptr, nullptr, h0, ht, o, cu_seqlens, state_indices, B,
                             T, Hqk, Hv, K, V, N, num_slots, scale, use_qk_l2norm, gate, stream,
                             name);
  return recurrent_plain(q, k, v, nullptr, nullptr, h0, ht, o, cu_seqlens, B, T, Hqk, Hv, K, V,
                         N, scale, use_qk_l2norm, gate, stream, name);
}

// Speculative decoding over a state pool (declared in gdn_layer.h): per-token
// states into the slots of a [N, index_stride] table, the initial state from
// the slot of the last accepted token.
extern "C" int gdn_recurrent_fwd_spec(const void* q, const void* k, const void* v,
                                      const float* g, const float* beta, float* pool, void* o,
                                      const int32_t* cu_seqlens, const int32_t* state_indices,
                                      int index_stride, const int32_t* num_accepted_tokens,
                                      int B, int T, int Hqk, int Hv, int K, int V, int N,
                                      int num_slots, float scale, int use_qk_l2norm,
                                      void* stream) {
  int rc = gdn_host::validate_common(q, k, v, g, beta, nullptr, nullptr, o, cu_seqlens, B, T,
                                     Hqk, Hv, K, V, N);
  if (rc) return rc;
  if (num_slots < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_recurrent_fwd_spec: num_slots must be >= 0");
  if (index_stride <= 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_recurrent_fwd_spec: index_stride must be > 0");
  if (!cu_seqlens && T > index_stride)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_recurrent_fwd_spec: T (" + std::to_string(T) +
                                             ") exceeds index_stride (" +
                                             std::to_string(index_stride) + ")");
  if (N > 0 && (!state_indices || !pool))
    return gdn_host::fail(GDN_ERR_NULL, "gdn_recurrent_fwd_spec: pool and state_indices must be non-NULL");
  if (N == 0 || num_slots == 0 || (long long)B * T == 0) return GDN_OK;
  gdn_host::launch_begin();
  auto* qq = static_cast<const uint16_t*>(q);
  auto* kk = static_cast<const uint16_t*>(k);
  auto* vv = static_cast<const uint16_t*>(v);
  auto* oo = static_cast<uint16_t*>(o);
  auto st = static_cast<hipStream_t>(stream);
#define GDN_RECS(KK, VV)                                                                    \
  if (K == KK && V == VV) {                                                                 \
    gdn::launch_recurrent<KK, VV>(qq, kk, vv, g, beta, pool, pool, oo, cu_seqlens, B, T, Hqk, \
                                  Hv, N, scale, use_qk_l2norm, state_indices, num_slots, st, \
                                  index_stride, num_accepted_tokens);                       \
    return gdn_host::check_launch("gdn_recurrent_fwd_spec");                                \
  }
  GDN_RECS(128, 128)
  GDN_RECS(64, 64)
  GDN_RECS(128, 64)
  GDN_RECS(64, 128)
#undef GDN_RECS
  return gdn_host::fail(GDN_ERR_SHAPE, "gdn_recurrent_fwd_spec: unsupported K/V");
}
