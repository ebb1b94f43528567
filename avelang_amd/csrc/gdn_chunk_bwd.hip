// Chunked gated-delta-rule BACKWARD for gfx950 (chunk = 64 tokens).
//
// The reference repository has no gated delta rule (forward or backward);
// the operator is FLA's chunk_gated_delta_rule, whose forward semantics are
// transformers modeling_qwen3_next.py:374-453.  The gradient below is
// reverse-mode differentiation of the chunked forward of gdn_chunk.hip.
//
// Per chunk c (rows i, j in [0, 64), c' = scale, S = state at the chunk's
// start, dS' = dL/d(state at its end) from later chunks):
//   d     = Tb (V - e^G * (K S))                 (forward: the per-token delta)
//   dd    = P^T dO + e^(G_L - G) * (K dS')       (dL/dd; P carries c')
//   Z     = Tb^T dd
//   dS    = e^G_L dS' - K^T (e^G * Z) + Q^T (c' e^G * dO)
// and every gradient of the chunk is local given S, dS', d and dd.
//
// Launches (after the forward's chunk table + prep in backward mode, which
// also writes T and the fragments of Tb^T, P^T and Q^T, and the forward
// chain in save mode, which stores S at every chunk start and d):
//   chunk_rev_sw_kernel (gdn_chunk_rev.hip) one workgroup per (sequence,
//                       v-head, 16-column V tile), reverse over the
//                       sequence's chunks; dS' in one wave's VGPRs (fp32),
//                       hi+lo splits where a product feeds dS (as the forward
//                       chain); stores dS' of every chunk and dd (bf16) and dh0
//   chunk_grad_kernel   one resident workgroup per CU, taking (chunk,
//                       qk-head) items in turn, fully parallel: the local
//                       gradients of the group's v-heads, dq / dk summed over
//                       the group in registers
#include <algorithm>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

struct BwdWs {
  ChunkWs f;              // forward workspace (gate, fragments, T, hs, dl, ...)
  uint16_t* dse;          // [NC][Hv][V][K] bf16: dL/d(end state) of every chunk, transposed
  uint16_t* dd;           // [NC][Hv][V/8][64][8] bf16: dL/dd, per chunk in column
                          // groups of 8 (rows past the sequence end 0)
};

// --------------------------------------------------- gradient kernel ----
// A workgroup of 8 waves works on one (chunk, qk-head) item at a time.
// Wave w8 owns row tile
// rt = w8 % 4 (chunk rows 16rt..16rt+15) and the column tiles of parity
// hf = w8 / 4 of every [64 x *] result.  "OL" = the MFMA output layout:
// lane (r16, grp) holds rows 16rt + 4grp + r (r = 0..3) of column 16ct + r16.
//
// Local gradients of one (chunk, v-head) given S (chunk start state), dS'
// (gradient into its end state), d and dd (all bf16 from the chains):
//   R1 = dO S^T, R2 = dd S^T, dKt = d dS'^T
//   dPt = lower_incl(c' dO d^T),  dT = dd (bV)^T - R2 (b e^G K)^T
//   dA = strict_lower(-T^T dT T^T)                       (fp32 MFMA)
//   M = dA * b_i Gam,  MP = dPt * Gam
//   dq = c' e^G R1 + MP K
//   dk = e^(G_L - G) dKt + b e^G (T^T dW) + M K + M^T K + MP^T Q,  dW = -R2
//   dv = b (T^T dd)
//   dbeta = V . (T^T dd) + e^G K . (T^T dW) + rowsum(dA KK Gam)
//   dG = c' e^G Q.R1 - rho + b e^G K.(T^T dW) + rowsum(X) - colsum(X)
//        (+ e^G_L <S, dS'> + sum(rho) on the last row),
//   X = (b_i dA KK + dPt QK) Gam,  rho_j = e^(G_L - G_j) K_j . dKt_j
//   dg = reverse cumsum of dG within the chunk.
// (c' is folded into dO: dPt and R1 use c' dO.)  V . (T^T dd) is formed as
// the column sums of T * (dd V^T), since (T^T dd)_i . V_i = sum_j T_ji (dd V^T)_ji.
//
// Every operand read by rows (S, dS' by state rows; d, V by token rows)
// streams through a double-buffered LDS stage of 32 rows: slice s + 1 is
// written to the free stage before slice s is multiplied, while slice
// s + 3 is already requested into registers.
constexpr int kGradThreads = 512;

// Sum over the 16 lanes of a row (lanes 16 g .. 16 g + 15), every lane of
// the row receiving it: within quads (lane ^ 1, lane ^ 2), then the
// half-row mirror (lane i <- 7 - i) and the row mirror (lane i <- 15 - i),
// as DPP moves: no LDS traffic, unlike a shuffle.
__device__ __forceinline__ float row16_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true));
  return x;
}

// Sum over all 64 lanes (row sums, then the four row totals read from lanes
// 0, 16, 32, 48), the same value in every lane.
__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  const int xi = __builtin_bit_cast(int, x);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 48)));
}

// Suffix sums over the 64 lanes: lane i receives x_i + ... + x_63.  Within
// each 16-lane row by DPP row shifts to the left (lanes past the row's end
// read 0), then each row adds the totals of the rows above it (their first
// lanes, read with readlane).
__device__ __forceinline__ float suffix_sum(float x, int lane) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x101, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x102, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x104, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x108, 0xF, 0xF, true));
  const int xi = __builtin_bit_cast(int, x);
  const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 16));
  const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 32));
  const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 48));
  const int row = lane >> 4;
  const float above = row == 0 ? t1 + (t2 + t3) : (row == 1 ? t2 + t3 : (row == 2 ? t3 : 0.f));
  return x + above;
}

template <int K, int V>
__global__ __launch_bounds__(kGradThreads) void chunk_grad_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ qraw, const uint16_t* __restrict__ kraw,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dO,
    const float* __restrict__ beta, const int32_t* __restrict__ cu, int N, int T, int total,
    int Hqk, int Hv, int nchunks, float scale, int l2norm, BwdWs ws, uint16_t* __restrict__ dq,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, float* __restrict__ dg,
    float* __restrict__ dbeta) {
  constexpr int NTH = kGradThreads;
  constexpr int KT = K / 16, VT = V / 16, KB = K / 32, VB = V / 32;
  constexpr int KH = KT / 2, VH = VT / 2;   // column tiles per wave
  constexpr int LK = K + 8, LV = V + 8, LT = 68, LC = 72;
  constexpr int NSS = K / 32;          // slices of S / dS' (32 state rows each)
  constexpr int NSL = NSS + 2;         // + two slices of d / V (32 token rows each)
  // Slices stream in the order d / V token slices first, then the state
  // slices: a wave takes the A fragments of d for its rows from the token
  // slice that holds them, for the state slices' d dS'^T products.
  // Position i of the stream -> slice index (state slices 0..NSS-1, token
  // slice t = NSS + t).
  auto slice_at = [](int i) { return i < 2 ? NSS + i : i - 2; };
  constexpr int NPOS = 32 * V / 8;     // 16-byte positions of one matrix in a slice
  static_assert(NPOS <= NTH, "one staged position per thread");
  __shared__ __attribute__((aligned(16))) uint16_t Ks[64][LK];
  __shared__ __attribute__((aligned(16))) uint16_t Qs[64][LK];
  // stage of the streamed slices: state slices [buf][matrix][V rows][32 + 8
  // columns] (rows of S^T / dS'^T), token slices [buf][matrix][32 rows][LV]
  constexpr int LS = 40;
  constexpr int kStgBytes = (2 * 2 * V * LS * 2 > 2 * 2 * 32 * LV * 2) ? 2 * 2 * V * LS * 2
                                                                        : 2 * 2 * 32 * LV * 2;
  __shared__ __attribute__((aligned(16))) unsigned char StgRaw[kStgBytes];
  uint16_t (*StgS)[2][V][LS] = reinterpret_cast<uint16_t (*)[2][V][LS]>(StgRaw);
  // token buffer 1 sits at the top of the stage, clear of state buffer 0:
  // state slice 0 is written while token slice 1 is read
  constexpr int kTokBuf = 2 * 32 * LV * 2;
  static_assert(2 * V * LS * 2 <= kStgBytes - kTokBuf, "token buffer 1 must clear state buffer 0");
  uint16_t (*const Stg[2])[32][LV] = {
      reinterpret_cast<uint16_t (*)[32][LV]>(StgRaw),
      reinterpret_cast<uint16_t (*)[32][LV]>(StgRaw + kStgBytes - kTokBuf)};
  __shared__ __attribute__((aligned(16))) float T32[64][LT];
  __shared__ __attribute__((aligned(16))) float X32[64][LT];
  __shared__ __attribute__((aligned(16))) uint16_t Tb16[64][LC];
  // dd rows and R2 (bf16) for the T^T products; reused for M and MP after
  constexpr int kRegA = 64 * LV * 2, kRegB = 64 * LK * 2;
  static_assert(kRegA >= 64 * LC * 2 && kRegB >= 64 * LC * 2, "M / MP alias dd / R2");
  __shared__ __attribute__((aligned(16))) unsigned char regA[kRegA];
  __shared__ __attribute__((aligned(16))) unsigned char regB[kRegB];
  uint16_t (*dds)[LV] = reinterpret_cast<uint16_t (*)[LV]>(regA);
  // R2, M and MP are kept transposed (row = column of the matrix), so that a
  // lane's four output-layout values (4 rows, one column) are one 8-byte write
  constexpr int LR = 68;   // row stride of R2^T (K rows of 64 tokens)
  static_assert(K * LR * 2 <= kRegB, "R2^T must fit in regB");
  uint16_t (*R2t)[LR] = reinterpret_cast<uint16_t (*)[LR]>(regB);
  uint16_t (*Mt)[LC] = reinterpret_cast<uint16_t (*)[LC]>(regB);
  uint16_t (*MPt)[LC] = reinterpret_cast<uint16_t (*)[LC]>(regA);
  __shared__ __attribute__((aligned(16))) float Gs[64];
  __shared__ __attribute__((aligned(16))) float Bs[64];
  // column partial sums over each row tile's 16 rows: of X (0) and of
  // T * (dd V^T) (1)
  __shared__ __attribute__((aligned(16))) float ColP[2][4][64];
  __shared__ __attribute__((aligned(16))) float RowP[2][5][64];   // row partials per half
  __shared__ float Red[8];

  const int Gn = Hv / Hqk;
  const int tid = threadIdx.x;

  // Work items (chunk, qk-head): item x is chunk x % nchunks of qk-head
  // x / nchunks, and a workgroup takes items x = blockIdx.x + j gridDim.x, so
  // that it stays resident and requests its next item's first operands
  // during the current item's last v-head.  A varlen item past the last
  // chunk is empty and skipped.
  struct Item {
    int ci, hq, t0, L;
  };
  const int nitems = nchunks * Hqk;
  auto find_item = [&](int& x, Item& it) -> bool {
    for (; x < nitems; x += gridDim.x) {
      const int ci = x % nchunks;
      int n, cfirst;
      if (cu) {
        const int32_t* off = ws.f.off;
        if (ci >= off[N]) continue;
        int lo = 0, hi = N;
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (off[mid] <= ci) lo = mid; else hi = mid;
        }
        n = lo;
        cfirst = off[n];
      } else {
        const int nct = (T + kChunk - 1) / kChunk;
        n = ci / nct;
        cfirst = n * nct;
      }
      int s, e;
      seq_bounds(cu, n, T, total, s, e);
      it.ci = ci;
      it.hq = x / nchunks;
      it.t0 = s + (ci - cfirst) * kChunk;
      it.L = min(kChunk, e - it.t0);
      return true;
    }
    return false;
  };
  int x = blockIdx.x;
  Item cur;
  if (!find_item(x, cur)) return;
  // the item being worked on (read by the v-head body and the dq / dk stores)
  int ci = cur.ci, hq = cur.hq, t0 = cur.t0, L = cur.L;
  int qkbytes = 0, vbytes = 0;

  // K / Q rows of an item's chunk (rows >= L read as zero) into Ks / Qs,
  // through registers: requested by load_kq, written by store_kq
  constexpr int NQ = 64 * K / 8 / NTH;   // 16-byte chunks per thread
  auto load_kq = [&](const Item& it, bool live, u16x8 (&kr)[NQ], u16x8 (&qr)[NQ]) {
    int tid = threadIdx.x;   // (re-formed per call: see the v-head body)
    asm volatile("" : "+v"(tid));
    const int nb = live ? it.L * Hqk * K * 2 : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(k + ((size_t)it.t0 * Hqk + it.hq) * K), 0, nb, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(q + ((size_t)it.t0 * Hqk + it.hq) * K), 0, nb, kBufferFlags);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int idx = tid + NTH * i, r = idx / (K / 8), c8 = 8 * (idx % (K / 8));
      const int off = (r * Hqk * K + c8) * 2;
      kr[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
      qr[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
    }
  };
  auto store_kq = [&](const u16x8 (&kr)[NQ], const u16x8 (&qr)[NQ]) {
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int idx = tid + NTH * i, r = idx / (K / 8), c8 = 8 * (idx % (K / 8));
      *reinterpret_cast<u16x8*>(&Ks[r][c8]) = kr[i];
      *reinterpret_cast<u16x8*>(&Qs[r][c8]) = qr[i];
    }
  };
  // the upper 16 x 16 blocks of T (zero, not stored in the workspace): set
  // once here, the v-heads write only the lower blocks
#pragma unroll
  for (int i = 0; i < 64 * 16 / NTH; ++i) {
    const int idx = tid + NTH * i, r = idx / 16, c4 = 4 * (idx % 16);
    if (c4 / 16 > r / 16) {
      *reinterpret_cast<f32x4*>(&T32[r][c4]) = zero4();
      *reinterpret_cast<u16x4*>(&Tb16[r][c4]) = u16x4{0, 0, 0, 0};
    }
  }

  f32x4 dQa[KH], dKa[KH];   // column tiles 2m + hf

  // Operands of a v-head's staging phase (slices 0..2 of S / dS' or d / V,
  // T, the dd rows, G and beta, the A fragments of dO), requested
  // into registers: for the first item's first v-head before the loop, for
  // every later v-head (of this item or the next) before the previous
  // v-head's dK / dQ products, so their latency overlaps that v-head's last
  // phases instead of opening the next one.  live = false (no next item)
  // requests them from empty resources.
  // T arrives as its 10 lower 16 x 16 blocks (1 KB each): wave w loads block
  // w, waves 0 and 1 also blocks 8 and 9
  static_assert(NTH == 512 && kTBlocks == 10, "one T block per wave, two more for waves 0, 1");
  constexpr int NT = 2, ND = 64 * V / 8 / NTH;
  u16x8 pre[3][2];
  f32x4 tv[NT];
  u16x8 dv8[ND];
  u16x8 aO[VB];
  float gsv = 0.f, bsv = 0.f;
  auto issue_stage = [&](const Item& it, int gi_t, bool live) {
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int ci = it.ci, t0 = it.t0, L = it.L, hq = it.hq;
    const int vbytes = live ? L * Hv * V * 2 : 0;
    const int lane = tid % 64;
    const int rt = __builtin_amdgcn_readfirstlane(tid / 64) & 3;
    const int r16 = lane % 16, grp = lane / 16;
    const int rowA = 16 * rt + r16;
    const int sp_r = (tid % NPOS) / (V / 8), sp_c8 = 8 * (tid % (V / 8));
    const int ss_v = (tid % NPOS) / 4, ss_k = 8 * (tid % 4);
    const int sp_vs = (ss_v * K + ss_k) * 2;
    const int sp_vt = (sp_r * Hv * V + sp_c8) * 2;
    const int sp_dl = ((sp_c8 >> 3) * 64 + sp_r) * 16;
    const int h = hq * Gn + gi_t;
    const size_t ch = (size_t)ci * Hv + h;
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        ws.f.hs + ch * K * V, 0, live ? K * V * 2 : 0, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rE = __builtin_amdgcn_make_buffer_rsrc(
        ws.dse + ch * K * V, 0, live ? K * V * 2 : 0, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rT = __builtin_amdgcn_make_buffer_rsrc(
        ws.f.tmat + ch * kTPacked, 0, live ? kTPacked * 4 : 0, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rdd = __builtin_amdgcn_make_buffer_rsrc(
        ws.dd + ch * 64 * V, 0, live ? 64 * V * 2 : 0, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rdl = __builtin_amdgcn_make_buffer_rsrc(
        ws.f.dl + ch * 64 * V, 0, live ? 64 * V * 2 : 0, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rdo = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(dO + ((size_t)t0 * Hv + h) * V), 0, vbytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(v + ((size_t)t0 * Hv + h) * V), 0, vbytes, kBufferFlags);
    if (tid < NPOS) {
#pragma unroll
      for (int i = 0; i < 3 && i < NSL; ++i) {
        const int sl = slice_at(i);
        if (sl < NSS) {
          const int so = 32 * sl * 2;
          pre[i][0] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rS, sp_vs, so, 0));
          pre[i][1] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rE, sp_vs, so, 0));
        } else {
          const int so = 32 * (sl - NSS) * Hv * V * 2;
          pre[i][0] = __builtin_bit_cast(
              u16x8, __builtin_amdgcn_raw_buffer_load_b128(rdl, sp_dl, 32 * (sl - NSS) * 16, 0));
          pre[i][1] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, sp_vt, so, 0));
        }
      }
    }
    {
      const int w = __builtin_amdgcn_readfirstlane(tid / 64);
      tv[0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rT, 16 * lane, 1024 * w, 0));
      if (w < 2)
        tv[1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rT, 16 * lane, 1024 * (8 + w), 0));
    }
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      // 16-byte chunk idx: token row idx % 64 of column group idx / 64
      const int idx = tid + NTH * i;
      dv8[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rdd, idx * 16, 0, 0));
    }
    if (tid < 64) {
      gsv = ws.f.gate[ch * 64 + tid];
      bsv = tid < L ? beta[(size_t)(t0 + min(tid, L - 1)) * Hv + h] : 0.f;
    }
#pragma unroll
    for (int b = 0; b < VB; ++b) {
      const int off = (rowA * Hv * V + 32 * b + 8 * grp) * 2;
      aO[b] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rdo, off, 0, 0));
    }
  };
  // One v-head of the group; prefetch() requests the next v-head's operands
  // (of this item or the next).  It is made unconditionally: a conditional
  // one keeps the previous operands live through the whole v-head for the
  // path that skips it, which spills.
  auto vhead = [&](int gi, auto prefetch, auto after_dk) {
    // The lane index is passed through an empty asm statement once per
    // v-head, so the many per-lane LDS / buffer addresses derived from it are
    // formed inside the loop where they are used, instead of being hoisted
    // out of it (live across the whole loop they exceed the register file and
    // spill; the spill reloads then wait on every outstanding store).
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid % 64;
    const int w8 = __builtin_amdgcn_readfirstlane(tid / 64);
    const int rt = w8 & 3, hf = w8 >> 2;
    const int r16 = lane % 16, grp = lane / 16;
    const int rowA = 16 * rt + r16;
    const int row0 = 16 * rt + 4 * grp;
    // staged position of this thread in a slice (both matrices)
    const bool stager = tid < NPOS;
    // token slice position: row sp_r, columns sp_c8..+7; state slice
    // position: S^T row ss_v, state columns ss_k..+7 of the slice
    const int sp_r = (tid % NPOS) / (V / 8), sp_c8 = 8 * (tid % (V / 8));
    const int ss_v = (tid % NPOS) / 4, ss_k = 8 * (tid % 4);
    const int sp_vs = (ss_v * K + ss_k) * 2;             // byte offset in a state slice
    const int sp_vt = (sp_r * Hv * V + sp_c8) * 2;       // byte offset in a token slice
    const int sp_dl = ((sp_c8 >> 3) * 64 + sp_r) * 16;   // the same in the chunk's d block
    const int h = hq * Gn + gi;
    const size_t ch = (size_t)ci * Hv + h;
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        ws.f.hs + ch * K * V, 0, K * V * 2, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rE = __builtin_amdgcn_make_buffer_rsrc(
        ws.dse + ch * K * V, 0, K * V * 2, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rdl = __builtin_amdgcn_make_buffer_rsrc(
        ws.f.dl + ch * 64 * V, 0, 64 * V * 2, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(v + ((size_t)t0 * Hv + h) * V), 0, vbytes, kBufferFlags);

    // slice sl: state columns 32 sl..32 sl + 31 of every row of S^T (matrix
    // 0) and dS'^T (matrix 1) for sl < NSS (both stored transposed, [V][K]),
    // token rows 32 (sl - NSS).. of d (0) and V (1) after; load_slice and
    // store_slice take the stream position i (slice slice_at(i), stage
    // buffer i % 2)
    float sde = 0.f;   // partial <S, dS'> of the positions this thread stages
    auto load_slice = [&](int i, u16x8 (&buf)[2]) {
      if (!stager) return;
      const int sl = slice_at(i);
      if (sl < NSS) {
        const int so = 32 * sl * 2;
        buf[0] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rS, sp_vs, so, 0));
        buf[1] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rE, sp_vs, so, 0));
      } else {
        const int so = 32 * (sl - NSS) * Hv * V * 2;
        buf[0] = __builtin_bit_cast(
            u16x8, __builtin_amdgcn_raw_buffer_load_b128(rdl, sp_dl, 32 * (sl - NSS) * 16, 0));
        buf[1] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, sp_vt, so, 0));
      }
    };
    auto store_slice = [&](int i, const u16x8 (&buf)[2]) {
      if (!stager) return;
      const int sl = slice_at(i);
      if (sl < NSS) {
        *reinterpret_cast<u16x8*>(&StgS[i & 1][0][ss_v][ss_k]) = buf[0];
        *reinterpret_cast<u16x8*>(&StgS[i & 1][1][ss_v][ss_k]) = buf[1];
      } else {
        *reinterpret_cast<u16x8*>(&Stg[i & 1][0][sp_r][sp_c8]) = buf[0];
        *reinterpret_cast<u16x8*>(&Stg[i & 1][1][sp_r][sp_c8]) = buf[1];
      }
      if (sl < NSS) {
        // bf16 pairs straight into v_dot2_f32_bf16.  Each pair passes an
        // empty asm statement of its own: bound as whole vectors instead,
        // this compiler fed the first pair's registers to all four products.
        const u32x4 a = __builtin_bit_cast(u32x4, buf[0]), b = __builtin_bit_cast(u32x4, buf[1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          unsigned int aj = a[j], bj = b[j];
          asm("" : "+v"(aj));
          asm("" : "+v"(bj));
          sde = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, aj),
                                                __builtin_bit_cast(bf16x2, bj), sde, false);
        }
      }
    };

    // ---- staging: the operands issue_stage() requested for this v-head
    __builtin_amdgcn_sched_barrier(0);
    store_slice(0, pre[0]);
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if (i == 0 || w8 < 2) {
        const int bi = i == 0 ? w8 : 8 + w8;
        const int brt = tmat_block_row(bi), bcb = bi - tmat_block(brt, 0);
        const int r = 16 * brt + lane / 4, c4 = 16 * bcb + 4 * (lane % 4);
        *reinterpret_cast<f32x4*>(&T32[r][c4]) = tv[i];
        *reinterpret_cast<u16x4*>(&Tb16[r][c4]) = f2bf4(tv[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int idx = tid + NTH * i, r = idx % 64, c8 = 8 * (idx / 64);
      *reinterpret_cast<u16x8*>(&dds[r][c8]) = dv8[i];
    }
    if (tid < 64) {
      Gs[tid] = gsv;
      Bs[tid] = bsv;
    }
    __syncthreads();

    // A fragments of dd (this wave's rows) from the staged dd rows
    u16x8 aD[VB];
#pragma unroll
    for (int b = 0; b < VB; ++b) aD[b] = *reinterpret_cast<const u16x8*>(&dds[rowA][32 * b + 8 * grp]);
    // row factors of this lane's OL rows
    const float GL = Gs[L - 1];
    f32x4 eg, dec, bt;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      eg[r] = __expf(Gs[row0 + r]);
      dec[r] = __expf(GL - Gs[row0 + r]);
      bt[r] = Bs[row0 + r];
    }
    f32x4 qr1 = zero4(), rho = zero4(), ktw = zero4();

    // ---- streamed products over the slices (this wave: column tile hf of
    // each slice)
    f32x4 dpt[2], ddv[2];
    u16x8 aL[VB];   // A fragments of d (this wave's rows), from its token slice
#pragma unroll
    for (int i = 0; i < NSL; ++i) {
      const int sl = slice_at(i);
      if (i + 1 < NSL) store_slice(i + 1, pre[(i + 1) % 3]);
      if (i + 3 < NSL) load_slice(i + 3, pre[(i + 3) % 3]);
      __builtin_amdgcn_sched_barrier(0);
      const int bufi = i & 1;
      if (sl >= NSS && (rt >> 1) == sl - NSS) {
#pragma unroll
        for (int b = 0; b < VB; ++b)
          aL[b] = *reinterpret_cast<const u16x8*>(&Stg[bufi][0][16 * (rt & 1) + r16][32 * b + 8 * grp]);
      }
      f32x4 x0 = zero4(), x1 = zero4(), x2 = zero4();
#pragma unroll
      for (int b = 0; b < VB; ++b) {
        // B[k = v][n = state column 16 hf + r16]: columns of the staged S^T /
        // dS'^T rows; B[k = v][n = token row 16 hf + r16]: staged d / V rows
        const u16x8 b0 = sl < NSS
            ? lds_colfrag(&StgS[bufi][0][0][0], LS, 32 * b, 16 * hf, lane)
            : *reinterpret_cast<const u16x8*>(&Stg[bufi][0][16 * hf + r16][32 * b + 8 * grp]);
        const u16x8 b1 = sl < NSS
            ? lds_colfrag(&StgS[bufi][1][0][0], LS, 32 * b, 16 * hf, lane)
            : *reinterpret_cast<const u16x8*>(&Stg[bufi][1][16 * hf + r16][32 * b + 8 * grp]);
        if (sl < NSS) {
          x0 = mfma16(aO[b], b0, x0);    // dO S^T
          x1 = mfma16(aD[b], b0, x1);    // dd S^T
          x2 = mfma16(aL[b], b1, x2);    // d dS'^T
        } else {
          x0 = mfma16(aO[b], b0, x0);    // dO d^T
          x1 = mfma16(aD[b], b1, x1);    // dd V^T
        }
      }
      if (sl < NSS) {
        const int ct = 2 * sl + hf;
        // Q, K at this lane's OL rows row0 + r, column 16 ct + r16: one
        // transposing read of the group's 4 x 16 block each
        const u16x4 q4v = lds_tr16(&Qs[row0 + (r16 >> 2)][16 * ct + 4 * (r16 & 3)]);
        const u16x4 k4v = lds_tr16(&Ks[row0 + (r16 >> 2)][16 * ct + 4 * (r16 & 3)]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float qv = bf2f(q4v[r]);
          const float kv = bf2f(k4v[r]);
          const float a = scale * x0[r];
          dQa[sl][r] += eg[r] * a;
          qr1[r] += qv * a;
          const float d2 = dec[r] * x2[r];
          dKa[sl][r] += d2;
          rho[r] += kv * d2;
        }
        *reinterpret_cast<u16x4*>(&R2t[16 * ct + r16][row0]) = f2bf4(x1);
      } else {
        dpt[sl - NSS] = x0;
        ddv[sl - NSS] = x1;
      }
      __syncthreads();
    }

    // ---- dT = dd (bV)^T - R2 (b e^G K)^T  -> X32 (fp32), tiles 2m + hf
    {
      u16x8 a2[KB];
#pragma unroll
      for (int b = 0; b < KB; ++b) a2[b] = lds_colfrag(&R2t[0][0], LR, 32 * b, 16 * rt, lane);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int ct = 2 * m + hf;
        f32x4 t2 = zero4();
#pragma unroll
        for (int b = 0; b < KB; ++b)
          t2 = mfma16(a2[b], *reinterpret_cast<const u16x8*>(&Ks[16 * ct + r16][32 * b + 8 * grp]), t2);
        const int j = 16 * ct + r16;
        const float bj = Bs[j], bgj = bj * __expf(Gs[j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) X32[row0 + r][j] = ddv[m][r] * bj - t2[r] * bgj;
      }
    }
    // ---- T^T dd (-> dv) and T^T dW = -T^T R2 (-> dk, dbeta, dG)
    {
      u16x8 ta[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) ta[b] = lds_colfrag(&Tb16[0][0], LC, 32 * b, 16 * rt, lane);
      const __amdgpu_buffer_rsrc_t rdv = __builtin_amdgcn_make_buffer_rsrc(
          dv + ((size_t)t0 * Hv + h) * V, 0, vbytes, kBufferFlags);
#pragma unroll
      for (int m = 0; m < VH; ++m) {
        const int ct = 2 * m + hf;
        f32x4 tu = zero4();
#pragma unroll
        for (int b = 0; b < 2; ++b)
          tu = mfma16(ta[b], lds_colfrag(&dds[0][0], LV, 32 * b, 16 * ct, lane), tu);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          __builtin_amdgcn_raw_buffer_store_b16(f2bf(bt[r] * tu[r]), rdv,
                                                ((row0 + r) * Hv * V + 16 * ct + r16) * 2, 0, 0);
      }
#pragma unroll
      for (int m = 0; m < KH; ++m) {
        const int ct = 2 * m + hf;
        f32x4 tw = zero4();
#pragma unroll
        for (int b = 0; b < 2; ++b)
          tw = mfma16(ta[b], cat8(*reinterpret_cast<const u16x4*>(&R2t[16 * ct + r16][32 * b + 8 * grp]),
                                  *reinterpret_cast<const u16x4*>(&R2t[16 * ct + r16][32 * b + 8 * grp + 4])),
                      tw);
        const u16x4 k4v = lds_tr16(&Ks[row0 + (r16 >> 2)][16 * ct + 4 * (r16 & 3)]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = -tw[r];   // (T^T dW)
          dKa[m][r] += bt[r] * eg[r] * x;
          ktw[r] += bf2f(k4v[r]) * x;
        }
      }
    }
    __syncthreads();   // X32 = dT complete; dd / R2 no longer needed

    // ---- dA = strict_lower(-T^T (dT T^T)) on fp32 MFMA (T lower triangular).
    // In step s of a 16-deep block q, lane (r16, grp) supplies k = 16 q +
    // 4 grp + s, so its four A or B values of a block are one float4 of a row.
    f32x4 m1[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int ct = 2 * m + hf;
      m1[m] = zero4();
      for (int q = 0; q <= ct; ++q) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&X32[rowA][16 * q + 4 * grp]);
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&T32[16 * ct + r16][16 * q + 4 * grp]);
#pragma unroll
        for (int st = 0; st < 4; ++st) m1[m] = mfma4f32(a4[st], b4[st], m1[m]);
      }
    }
    __syncthreads();
    // M1 goes back transposed (X32 then holds M1^T): a lane's 4 output-layout
    // rows of column 16 ct + r16 are one float4
#pragma unroll
    for (int m = 0; m < 2; ++m)
      *reinterpret_cast<f32x4*>(&X32[16 * (2 * m + hf) + r16][row0]) = m1[m];
    __syncthreads();
    f32x4 da[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int ct = 2 * m + hf;
      da[m] = zero4();
      if (ct <= rt) {
        for (int q = rt; q < 4; ++q) {
          // B[k][n] = M1[k][16 ct + n] = M1^T[16 ct + n][k]
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(&X32[16 * ct + r16][16 * q + 4 * grp]);
#pragma unroll
          for (int st = 0; st < 4; ++st)
            da[m] = mfma4f32(T32[16 * q + 4 * grp + st][rowA], b4[st], da[m]);
        }
      }
    }
    // (no barrier here: the phases up to the next one write only Mt / MPt
    // (regB / regA, free since the T^T products) and ColP)

    // ---- K K^T and Q K^T (OL, this wave's two column tiles)
    f32x4 kk[2], qk[2];
    {
      u16x8 ka[KB], qa[KB];
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        ka[b] = *reinterpret_cast<const u16x8*>(&Ks[rowA][32 * b + 8 * grp]);
        qa[b] = *reinterpret_cast<const u16x8*>(&Qs[rowA][32 * b + 8 * grp]);
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int ct = 2 * m + hf;
        kk[m] = zero4();
        qk[m] = zero4();
#pragma unroll
        for (int b = 0; b < KB; ++b) {
          const u16x8 kb = *reinterpret_cast<const u16x8*>(&Ks[16 * ct + r16][32 * b + 8 * grp]);
          kk[m] = mfma16(ka[b], kb, kk[m]);
          qk[m] = mfma16(qa[b], kb, qk[m]);
        }
      }
    }
    // ---- C x C elementwise: M, MP, dbeta / dG terms, the column sums of X and T * (dd V^T)
    f32x4 dba = zero4(), xr = zero4();
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int j = 16 * (2 * m + hf) + r16;
      const float Gj = Gs[j];
      f32x4 mv, mpv;
      float xc = 0.f, tc = 0.f;   // column j over this lane's 4 rows
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = row0 + r;
        const float gam = (j <= i) ? __expf(Gs[i] - Gj) : 0.f;
        const float dA = (j < i) ? -da[m][r] : 0.f;
        const float dP = (j <= i) ? scale * dpt[m][r] : 0.f;
        mv[r] = dA * bt[r] * gam;
        mpv[r] = dP * gam;
        dba[r] += dA * kk[m][r] * gam;
        const float x = (dA * bt[r] * kk[m][r] + dP * qk[m][r]) * gam;
        xr[r] += x;
        xc += x;
        tc += T32[i][j] * ddv[m][r];   // T_ij (dd V^T)_ij
      }
      *reinterpret_cast<u16x4*>(&Mt[j][row0]) = f2bf4(mv);
      *reinterpret_cast<u16x4*>(&MPt[j][row0]) = f2bf4(mpv);
      // over the row tile's 16 rows (the wave's 4 lane groups): one partial
      // per (row tile, column)
      xc += __shfl_xor(xc, 16);
      xc += __shfl_xor(xc, 32);
      tc += __shfl_xor(tc, 16);
      tc += __shfl_xor(tc, 32);
      if (grp == 0) {
        ColP[0][rt][j] = xc;
        ColP[1][rt][j] = tc;
      }
    }
    __syncthreads();   // M, MP complete

    prefetch();

    // ---- dK += M K + M^T K + MP^T Q,  dQ += MP K (this wave's column tiles)
    {
      u16x8 am[2], amt[2], ap[2], apt[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        am[b] = lds_colfrag(&Mt[0][0], LC, 32 * b, 16 * rt, lane);
        ap[b] = lds_colfrag(&MPt[0][0], LC, 32 * b, 16 * rt, lane);
        amt[b] = *reinterpret_cast<const u16x8*>(&Mt[rowA][32 * b + 8 * grp]);
        apt[b] = *reinterpret_cast<const u16x8*>(&MPt[rowA][32 * b + 8 * grp]);
      }
#pragma unroll
      for (int m = 0; m < KH; ++m) {
        const int ct = 2 * m + hf;
        f32x4 a0 = dKa[m], a1 = zero4(), a2 = dQa[m];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const u16x8 kc = lds_colfrag(&Ks[0][0], LK, 32 * b, 16 * ct, lane);
          const u16x8 qc = lds_colfrag(&Qs[0][0], LK, 32 * b, 16 * ct, lane);
          a0 = mfma16(am[b], kc, a0);
          a1 = mfma16(amt[b], kc, a1);
          a1 = mfma16(apt[b], qc, a1);
          a2 = mfma16(ap[b], kc, a2);
        }
        dKa[m] = a0 + a1;
        dQa[m] = a2;
      }
    }

    after_dk();

    // ---- row partials: reduce over the 16 lanes of a group, then combine
    // the two column halves through LDS
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      qr1[r] = row16_sum(qr1[r]);
      rho[r] = row16_sum(rho[r]);
      ktw[r] = row16_sum(ktw[r]);
      dba[r] = row16_sum(dba[r]);
      xr[r] = row16_sum(xr[r]);
    }
    if (r16 == 0) {
      *reinterpret_cast<f32x4*>(&RowP[hf][0][row0]) = qr1;
      *reinterpret_cast<f32x4*>(&RowP[hf][1][row0]) = rho;
      *reinterpret_cast<f32x4*>(&RowP[hf][2][row0]) = ktw;
      *reinterpret_cast<f32x4*>(&RowP[hf][3][row0]) = dba;
      *reinterpret_cast<f32x4*>(&RowP[hf][4][row0]) = xr;
    }
    sde = wave_sum(sde);
    if (lane == 0) Red[w8] = sde;
    __syncthreads();   // ColP, RowP, Red complete
    if (w8 == 0) {
      // per row (lane = row): total dG and dbeta, then dg = reverse cumsum
      const int i = lane;
      float sd = 0.f;
#pragma unroll
      for (int x = 0; x < 8; ++x) sd += Red[x];
      const float rq1 = RowP[0][0][i] + RowP[1][0][i];
      const float rrho = RowP[0][1][i] + RowP[1][1][i];
      const float rktw = RowP[0][2][i] + RowP[1][2][i];
      const float rdba = RowP[0][3][i] + RowP[1][3][i];
      const float rxr = RowP[0][4][i] + RowP[1][4][i];
      const float rho_all = wave_sum(rrho);
      float csum = 0.f, cvsum = 0.f;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        csum += ColP[0][x][i];
        cvsum += ColP[1][x][i];
      }
      const float egi = __expf(Gs[i]), bi = Bs[i];
      float dG = egi * rq1 - rrho + bi * egi * rktw + rxr - csum;
      if (i == L - 1) dG += __expf(GL) * sd + rho_all;
      if (i < L) dbeta[(size_t)(t0 + i) * Hv + h] = cvsum + egi * rktw + rdba;
      // dg = reverse inclusive cumsum of dG over the 64 rows
      const float x = suffix_sum(i < L ? dG : 0.f, lane);
      if (i < L) dg[(size_t)(t0 + i) * Hv + h] = x;
    }
    __syncthreads();   // LDS reuse by the next v-head
  };
  issue_stage(cur, 0, true);
  {
    u16x8 kr[NQ], qr[NQ];
    load_kq(cur, true, kr, qr);
    store_kq(kr, qr);
  }
  for (;;) {
    __syncthreads();
    ci = cur.ci;
    hq = cur.hq;
    t0 = cur.t0;
    L = cur.L;
    qkbytes = L * Hqk * K * 2;
    vbytes = L * Hv * V * 2;
#pragma unroll
    for (int m = 0; m < KH; ++m) {
      dQa[m] = zero4();
      dKa[m] = zero4();
    }
    int xn = x + gridDim.x;
    Item nxt;
    const bool more = find_item(xn, nxt);
    if (!more) nxt = cur;
    // the next item's K / Q rows are requested once the last v-head's dK / dQ
    // products are issued (their registers then free) and written to Ks / Qs
    // after this item's dq / dk stores (Ks / Qs free since the last v-head's
    // closing barrier; the wait for them counts none of those stores)
    u16x8 kr[NQ], qr[NQ];
    for (int gi = 0; gi + 1 < Gn; ++gi)
      vhead(gi, [&] { issue_stage(cur, gi + 1, true); }, [] {});
    vhead(Gn - 1, [&] { issue_stage(nxt, 0, more); }, [&] { load_kq(nxt, more, kr, qr); });

    // ---- dq, dk: through the l2norm when the forward normalised q, k
    // (the lane indices re-formed here, as in the v-head body, so that the
    // stores' per-lane offsets are not kept live across the item loop)
    {
      int tid = threadIdx.x;
      asm volatile("" : "+v"(tid));
      const int lane = tid % 64;
      const int hf = __builtin_amdgcn_readfirstlane(tid / 64) >> 2;
      const int r16 = lane % 16;
      const int row0 = 16 * (__builtin_amdgcn_readfirstlane(tid / 64) & 3) + 4 * (lane / 16);
      const __amdgpu_buffer_rsrc_t rdq = __builtin_amdgcn_make_buffer_rsrc(
          dq + ((size_t)t0 * Hqk + hq) * K, 0, qkbytes, kBufferFlags);
      const __amdgpu_buffer_rsrc_t rdk = __builtin_amdgcn_make_buffer_rsrc(
          dk + ((size_t)t0 * Hqk + hq) * K, 0, qkbytes, kBufferFlags);
      if (l2norm) {
        const __amdgpu_buffer_rsrc_t rqr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(qraw + ((size_t)t0 * Hqk + hq) * K), 0, qkbytes, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rkr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(kraw + ((size_t)t0 * Hqk + hq) * K), 0, qkbytes, kBufferFlags);
        f32x4 sq = zero4(), sk = zero4(), pq = zero4(), pk = zero4();
        float xq[KH][4], xk[KH][4];
#pragma unroll
        for (int m = 0; m < KH; ++m) {
          const int ct = 2 * m + hf;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int off = ((row0 + r) * Hqk * K + 16 * ct + r16) * 2;
            xq[m][r] = bf2f(__builtin_amdgcn_raw_buffer_load_b16(rqr, off, 0, 0));
            xk[m][r] = bf2f(__builtin_amdgcn_raw_buffer_load_b16(rkr, off, 0, 0));
            sq[r] += xq[m][r] * xq[m][r];
            sk[r] += xk[m][r] * xk[m][r];
            pq[r] += xq[m][r] * dQa[m][r];
            pk[r] += xk[m][r] * dKa[m][r];
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sq[r] = row16_sum(sq[r]);
          sk[r] = row16_sum(sk[r]);
          pq[r] = row16_sum(pq[r]);
          pk[r] = row16_sum(pk[r]);
        }
        // combine the two column halves (RowP is free after the v-head loop)
        if (r16 == 0) {
          *reinterpret_cast<f32x4*>(&RowP[hf][0][row0]) = sq;
          *reinterpret_cast<f32x4*>(&RowP[hf][1][row0]) = sk;
          *reinterpret_cast<f32x4*>(&RowP[hf][2][row0]) = pq;
          *reinterpret_cast<f32x4*>(&RowP[hf][3][row0]) = pk;
        }
        __syncthreads();
        // dx = r (dy - y (y . dy)), y = x r, r = (|x|^2 + eps)^-1/2
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = row0 + r;
          const float tq = RowP[0][0][i] + RowP[1][0][i], tk = RowP[0][1][i] + RowP[1][1][i];
          const float uq = RowP[0][2][i] + RowP[1][2][i], uk = RowP[0][3][i] + RowP[1][3][i];
          const float rq = rsqrtf(tq + 1e-6f), rk2 = rsqrtf(tk + 1e-6f);
#pragma unroll
          for (int m = 0; m < KH; ++m) {
            dQa[m][r] = rq * (dQa[m][r] - xq[m][r] * rq * rq * uq);
            dKa[m][r] = rk2 * (dKa[m][r] - xk[m][r] * rk2 * rk2 * uk);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < KH; ++m) {
        const int ct = 2 * m + hf;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int off = ((row0 + r) * Hqk * K + 16 * ct + r16) * 2;
          __builtin_amdgcn_raw_buffer_store_b16(f2bf(dQa[m][r]), rdq, off, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b16(f2bf(dKa[m][r]), rdk, off, 0, 0);
        }
      }
    }
    if (!more) break;
    store_kq(kr, qr);
    cur = nxt;
    x = xn;
  }
}

}  // namespace gdn

// ------------------------------------------------------------- host ----
namespace gdn {

template <int K, int V>
static void launch_bwd_kernels(const uint16_t* q, const uint16_t* k, const uint16_t* qn,
                               const uint16_t* kn, const uint16_t* v, const uint16_t* dO,
                               const float* beta, const float* dht, float* dh0,
                               const int32_t* cu, int B, int T, int Hqk, int Hv, int N,
                               float scale, bool l2, const WsPlan& p, unsigned char* wsb,
                               uint16_t* dq, uint16_t* dk, uint16_t* dv, float* dg,
                               float* dbeta, hipStream_t st) {
  BwdWs ws;
  ws.f = ws_pointers(p, wsb);
  ws.dse = reinterpret_cast<uint16_t*>(wsb + p.dse);
  ws.dd = reinterpret_cast<uint16_t*>(wsb + p.dd);
  const int total = B * T;
  launch_rev_sw<K>(dO, dht, dh0, cu, N, T, total, Hqk, Hv, V, scale, ws.f, ws.dse, ws.dd, st);
  if (p.ncmax > 0) {
    // one resident workgroup per CU (the kernel's LDS allows no second),
    // each taking every grid-th (chunk, qk-head) item
    const long long items = p.ncmax * (long long)Hqk;
    const int grid = (int)std::min<long long>(items, device_cus());
    hipLaunchKernelGGL((chunk_grad_kernel<K, V>), dim3(grid), dim3(kGradThreads), 0, st, qn, kn,
                       q, k, v, dO, beta, cu, N, T, total, Hqk, Hv, (int)p.ncmax, scale,
                       l2 ? 1 : 0, ws, dq, dk, dv, dg, dbeta);
  }
}

}  // namespace gdn

namespace gdn_host {
int validate_common(const void* q, const void* k, const void* v, const float* g,
                    const float* beta, const float* h0, const float* ht, const void* o,
                    const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N);
}

extern "C" size_t gdn_chunk_bwd_workspace_bytes(int B, int T, int Hqk, int Hv, int K, int V,
                                                int N, int has_cu_seqlens, int use_qk_l2norm) {
  if (B < 0 || T < 0 || Hqk <= 0 || Hv <= 0 || N < 0 || K <= 0 || V <= 0) return 0;
  return gdn::plan_ws(B, T, Hqk, Hv, K, V, N, has_cu_seqlens != 0, use_qk_l2norm != 0, true)
      .total;
}

extern "C" int gdn_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                             const float* beta, const float* h0, const void* dO,
                             const float* dht, void* dq, void* dk, void* dv, float* dg,
                             float* dbeta, float* dh0, const int32_t* cu_seqlens, int B, int T,
                             int Hqk, int Hv, int K, int V, int N, float scale,
                             int use_qk_l2norm, int saved, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = gdn_host::validate_common(q, k, v, g, beta, h0, nullptr, dO, cu_seqlens, B, T, Hqk,
                                     Hv, K, V, N);
  if (rc) return rc;
  const long long tokens = (long long)B * T;
  if (tokens > 0 && (!dq || !dk || !dv || !dg || !dbeta))
    return gdn_host::fail(GDN_ERR_NULL, "gdn_chunk_bwd: dq, dk, dv, dg and dbeta must be non-NULL");
  {
    // the gradients are written while the inputs are still being read: no
    // output may share memory with an input or with another output
    const size_t nqk = (size_t)tokens * Hqk * K * 2, nv = (size_t)tokens * Hv * V * 2;
    const size_t ng = (size_t)tokens * Hv * 4, ns = (size_t)N * Hv * K * V * 4;
    const void* in[] = {q, k, v, g, beta, h0, dO, dht};
    const size_t nin[] = {nqk, nqk, nv, ng, ng, h0 ? ns : 0, nv, dht ? ns : 0};
    const void* out[] = {dq, dk, dv, dg, dbeta, dh0};
    const size_t nout[] = {nqk, nqk, nv, ng, ng, dh0 ? ns : 0};
    for (int i = 0; i < 6; ++i) {
      for (int j = 0; j < 8; ++j)
        if (out[i] && in[j] && gdn_host::overlaps(out[i], nout[i], in[j], nin[j]))
          return gdn_host::fail(GDN_ERR_ALIAS, "gdn_chunk_bwd: a gradient buffer overlaps an input");
      for (int j = i + 1; j < 6; ++j)
        if (out[i] && out[j] && gdn_host::overlaps(out[i], nout[i], out[j], nout[j]))
          return gdn_host::fail(GDN_ERR_ALIAS, "gdn_chunk_bwd: two gradient buffers overlap");
    }
  }
  if (N == 0 || (tokens == 0 && !dh0)) return GDN_OK;
  gdn_host::launch_begin();
  const gdn::WsPlan p = gdn::plan_ws(B, T, Hqk, Hv, K, V, N, cu_seqlens != nullptr,
                                     use_qk_l2norm != 0, true);
  if (!workspace || workspace_bytes < p.total)
    return gdn_host::fail(GDN_ERR_WORKSPACE, "gdn_chunk_bwd: workspace needs " +
                                                 std::to_string(p.total) + " bytes, got " +
                                                 std::to_string(workspace_bytes));
  if (p.ncmax > (1LL << 30) || (long long)N * Hv * (V / 16) >= (1LL << 31) ||
      p.ncmax * (long long)Hqk >= (1LL << 30))
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_chunk_bwd: problem too large");
  auto* wsb = static_cast<unsigned char*>(workspace);
  auto st = static_cast<hipStream_t>(stream);
  auto* qq = static_cast<const uint16_t*>(q);
  auto* kk = static_cast<const uint16_t*>(k);
  auto* vv = static_cast<const uint16_t*>(v);
  const bool l2 = use_qk_l2norm != 0;
  // forward recomputation: prep (with T, Tb^T, P^T) and the chain saving the
  // chunk-start states and the deltas -- unless gdn_chunk_fwd_save already
  // left them in this workspace
  if (!saved)
    gdn::launch_chunk_fwd(qq, kk, vv, g, beta, h0, nullptr, nullptr, cu_seqlens, B, T, Hqk, Hv,
                          K, V, N, scale, l2, gdn::FwdMode::kRecompute, p, wsb, st);
  const uint16_t* qn = l2 ? reinterpret_cast<const uint16_t*>(wsb + p.qn) : qq;
  const uint16_t* kn = l2 ? reinterpret_cast<const uint16_t*>(wsb + p.kn) : kk;
  auto* ddo = static_cast<const uint16_t*>(dO);
  auto* dqq = static_cast<uint16_t*>(dq);
  auto* dkk = static_cast<uint16_t*>(dk);
  auto* dvv = static_cast<uint16_t*>(dv);
#define GDN_BWD(KK_, VV_)                                                                    \
  gdn::launch_bwd_kernels<KK_, VV_>(qq, kk, qn, kn, vv, ddo, beta, dht, dh0, cu_seqlens, B, T, \
                                    Hqk, Hv, N, scale, l2, p, wsb, dqq, dkk, dvv, dg, dbeta, st)
  if (K == 128 && V == 128) GDN_BWD(128, 128);
  else if (K == 128) GDN_BWD(128, 64);
  else if (V == 128) GDN_BWD(64, 128);
  else GDN_BWD(64, 64);
#undef GDN_BWD
  if (cu_seqlens) {
    // a cu_seqlens violation (found by the forward's chunk table, in this
    // workspace) left every sequence empty: the gradients are zero-filled
    // (and dh0 = dht, written by the reverse chain for an empty sequence)
    gdn::ZeroList z{};
    const size_t nqk = (size_t)tokens * Hqk * K * 2, nv = (size_t)tokens * Hv * V * 2;
    const size_t ng = (size_t)tokens * Hv * 4;
    void* outs[] = {dq, dk, dv, dg, dbeta};
    const size_t sizes[] = {nqk, nqk, nv, ng, ng};
    for (int i = 0; i < 5; ++i) {
      z.p[i] = outs[i];
      z.bytes[i] = sizes[i];
    }
    gdn::launch_zero_on_violation(gdn::ws_pointers(p, wsb).status, z, st);
  }
  return gdn_host::check_launch("gdn_chunk_bwd");
}
