// Forward chain of the chunked prefill, state-wave form (gfx950).
//
// One workgroup per (sequence, v-head, 16-column V tile) -- or per two V
// tiles when the chains fill the GPU twice over -- sequential over the
// sequence's chunks of 64 tokens:
//
//   the state wave (one per V tile) holds every key row of the tile's fp32
//   state in VGPRs and runs the serial part of a chunk step alone:
//       X = K S,  Y = V - e^G X,  vnew = Tb Y,
//       S = e^G_last S + K^T (e^(G_last - G) vnew)
//   (Tb = (I + A)^-1 diag(beta) from the prep kernel; K S, Tb Y and K^T U
//   as single fp16 MFMA products of operands rounded from fp32, which keeps
//   the final state within ~4e-4 relative Frobenius of the exact chain at
//   any length).  Each product's result tile is the next
//   product's B operand where it stands (row orders below), so no LDS
//   exchange sits inside the step, and every operand comes from LDS.
//
//   the stage wave loads chunk c+2's K rows (the prep kernel's fp16 copy,
//   already in this kernel's LDS layout), Tb fragments (already in rho row
//   order) and V tiles straight into LDS (buffer_load ... lds) while step c
//   runs.
//
//   two output waves form chunk c-1's output, two of its four 16-row tiles
//   each, from the state and vnew fragments the state waves leave in LDS:
//       o = scale e^G (Q S) + P vnew
//   and the first writes chunk c+1's gate factors into LDS (with both the
//   backward's saves and o, a save wave stores the former; without o, one
//   wave writes the gate factors and stores the saves).
//
// One s_barrier per chunk step hands the buffers over (three stage buffers,
// three output buffers).  The state wave issues no global load at all.
//
// Row orders.  An MFMA result tile puts rows 4 grp + r (r < 4) in lane
// (n, grp); a B operand of k-block b takes reduction slots 8 grp + i (i < 8)
// from lane (n, grp).  Tile row 16 T + 4 grp + r stands for index
//     rho(16 T + 4 grp + r) = 32 (T / 2) + 8 grp + 4 (T % 2) + r,
// so a lane's rows of tiles 2b and 2b + 1 are exactly the natural indices
// 32 b + 8 grp + i of k-block b.  The state's key rows and the token rows of
// X, Y and vnew use rho; K, Q, P and the columns of Tb stay in natural
// order (the prep writes the Tb fragments by rho-permuted row).
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

// SAVE: store the state at every chunk start (ws.hs, bf16, transposed) and
// the per-token delta vnew (ws.dl, bf16) for the backward.  OUT: write o and
// ht.  Forward <K, false, true>, the backward's recomputation <K, true,
// false>, a training forward <K, true, true>.  NS: V tiles (slices) per
// workgroup, one state wave each, sharing the stage wave's K / Tb buffers
// and the output waves' Q / P (2 when there are enough chains to fill the
// GPU twice over).
//
// Without use_qk_l2norm the chain reads the caller's bf16 rows where the
// prep kernel would otherwise have to copy them:
// RAWQ (forms with OUT): the output waves take Q S on bf16 MFMA, Q rows
//   loaded as they are and the state's fp16 fragments re-rounded to bf16 --
//   the rounding the operator's bf16 contract allows there, while the state's
//   own products keep fp16 (the prep writes no fp16 Q copy).  The state wave
//   publishes the same fp16 fragments in every form, so the backward's saved
//   states do not depend on it.
// RAWK (a plain forward, one V tile per workgroup): a fourth (convert) wave
//   loads chunk c+2's K rows into its registers during step c and writes
//   chunk c+1's, converted, as the fp16 KLayout block (rows past the
//   sequence end 0); the prep writes no fp16 K copy.  (The backward's chains
//   and two V tiles per workgroup keep the copy: the reverse chain reads it
//   too, and the convert wave's registers would not fit beside two state
//   waves.)  The output work is split over two waves as well (two o tiles
//   each), since with one output wave that wave set the step.
// Forms with o split the output work over two waves (the last role is the
// second output wave; before it come the convert wave with RAWK and the save
// wave with both outputs).
template <bool SAVE, bool OUT, int NS>
constexpr bool chain_split_out() { return OUT && (NS == 1 || !SAVE); }
template <bool SAVE, bool OUT, int NS, bool RAWK>
constexpr int chain_waves() {
  return NS + 2 + (SAVE && OUT ? 1 : 0) + (RAWK ? 1 : 0) + (chain_split_out<SAVE, OUT, NS>() ? 1 : 0);
}

template <int K, bool SAVE, bool OUT, int NS, bool RAWK, bool RAWQ>
__global__ __launch_bounds__((chain_waves<SAVE, OUT, NS, RAWK>() * 64)) void
chunk_chain_sw_kernel(const uint16_t* __restrict__ v, const uint16_t* __restrict__ qraw,
                      const uint16_t* __restrict__ kraw, const float* h0, float* ht,
                      uint16_t* __restrict__ o, const int32_t* __restrict__ cu, int N, int T,
                      int total, int Hqk, int Hv, int V, float scale, ChunkWs ws) {
  static_assert(!RAWK || (OUT && !SAVE && NS == 1 && RAWQ), "RAWK is a plain forward");
  static_assert(!RAWQ || OUT, "RAWQ forms o");
  static_assert(!OUT || chain_split_out<SAVE, OUT, NS>(), "every form with o splits its output");
  constexpr int KB = K / 32;   // k-blocks over the key index
  constexpr int ST = K / 16;   // 16-row state tiles
  // Stage buffers (chunk c in buffer c % 3): the chunk's K rows (KLayout),
  // the Tb A fragments in rho row order, the V tile as it sits in v (bf16,
  // [token][16 columns] per slice), e^G and e^(G_last - G) by token, and
  // e^G_last.
  using KL = KLayout<K>;
  __shared__ __attribute__((aligned(16))) unsigned char Kst[3][KL::BYTES];
  __shared__ __attribute__((aligned(16))) u16x8 Tst[3][6][64];
  __shared__ __attribute__((aligned(16))) uint16_t Vrw[3][NS][64][16];
  __shared__ __attribute__((aligned(16))) float Gst[3][2][64];
  __shared__ float Egl[3];
  // Output buffers (chunk c in buffer c % 3), left by the state wave for
  // the output waves: the state's hi B fragments at the chunk start and
  // vnew (bf16) as B fragments.
  __shared__ __attribute__((aligned(16))) u16x8 Sx[3][NS][KB][64];
  __shared__ __attribute__((aligned(16))) u16x8 Vx[3][NS][2][64];

  const int NVT = V / (16 * NS);   // workgroups per v-head
  // XCD-aware placement, as in the four-wave chain: a qk-head group's
  // workgroups stay on one XCD (shared K / Q / Tb / P in its L2), and the
  // groups are dealt round-robin so every XCD gets a share of each sequence.
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  const int unit = NVT * (Hv / Hqk);
  if (nb % (8 * unit) == 0) {
    const int i = bid >> 3;
    bid = ((i / unit) * 8 + (bid & 7)) * unit + i % unit;
  } else if ((nb & 7) == 0) {
    bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  }
  const int vt0 = (bid % NVT) * NS;   // first V tile of this workgroup
  const int h = (bid / NVT) % Hv;
  const int n = bid / NVT / Hv;
  const int hq = h / (Hv / Hqk);

  const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int r16 = lane % 16, grp = lane / 16;

  int s, e;
  seq_bounds(cu, n, T, total, s, e);
  const int nct = (T + kChunk - 1) / kChunk;
  const int c_begin = cu ? ws.off[n] : n * nct;
  const int nc = (cu ? ws.off[n + 1] : (n + 1) * nct) - c_begin;

  // the state wave of V tile `vs` (a compile-time index, so that its LDS
  // addresses are immediates as with one tile per workgroup)
  auto state_wave = [&](auto slc) {
    constexpr int vs = decltype(slc)::value;
    // ------------------------------------------------------ state wave ----
    const int vt = vt0 + vs;   // this wave's V tile
    // state tile t: lane (n16, grp), element r = S[rho(16t + 4grp + r)][16 vt + n16]
    const size_t tile = ((size_t)n * Hv + h) * (size_t)K * V + 16 * vt + r16;
    f32x4 S[ST];
    if (h0) {
#pragma unroll
      for (int t = 0; t < ST; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) S[t][r] = h0[tile + (size_t)rho_row(t, 4 * grp + r) * V];
      }
    } else {
#pragma unroll
      for (int t = 0; t < ST; ++t) S[t] = zero4();
    }
    __syncthreads();   // stage buffer 0 is filled

    // per-lane byte offsets into a K stage buffer (KLayout): K A fragments
    // of k-block b (row rho(16 ti + r16), unit 4 b + grp; tile ti adds
    // rows 32 (ti / 2) + 4 (ti % 2), which leave swz unchanged) and the
    // transposing reads of K^T for state tiles 2u, 2u + 1 (row 8 grp + m4,
    // unit 4 u + q4; the second 4 rows, k-block b's 32 rows and 8 (t % 2)
    // bytes are compile-time offsets)
    const int m4 = r16 >> 2, q4 = r16 & 3;
    int ka_off[KB], tr_off[ST / 2];
#pragma unroll
    for (int b = 0; b < KB; ++b) ka_off[b] = KL::off(rho_row(0, r16), 4 * b + grp);
#pragma unroll
    for (int u = 0; u < ST / 2; ++u) tr_off[u] = KL::off(8 * grp + m4, 4 * u + q4);

    // one chunk step on stage / output buffer B3 (a compile-time index, so
    // that every LDS address is a per-lane base plus an immediate)
    auto step = [&](auto b3c) {
      constexpr int b3 = decltype(b3c)::value;
      const unsigned char* Kb = Kst[b3];
      // operands of the step, all from LDS and issued first, in the order
      // they are used (e^G_last first: the state's decay may be scheduled
      // early)
      const float egl = Egl[b3];
      u16x8 ka[KB][4], ta[6];
#pragma unroll
      for (int b = 0; b < KB; ++b) {
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
          ka[b][ti] = *reinterpret_cast<const u16x8*>(
              Kb + ka_off[b] + KL::RS * (32 * (ti >> 1) + 4 * (ti & 1)));
      }
#pragma unroll
      for (int i = 0; i < 6; ++i) ta[i] = Tst[b3][i][lane];
      // V at tokens rho(16 ti + 4 grp + r) = r0 + r, column r16: one
      // transposing read of the 4 token rows per tile (widened to fp32 only
      // where Y is formed, so that no read waits on another's conversion)
      f32x4 eg[4], dc[4];
      u16x4 v4[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int r0 = 32 * (ti >> 1) + 8 * grp + 4 * (ti & 1);
        v4[ti] = lds_tr16(&Vrw[b3][vs][r0 + (r16 >> 2)][4 * (r16 & 3)]);
      }
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int r0 = 32 * (ti >> 1) + 8 * grp + 4 * (ti & 1);
        eg[ti] = *reinterpret_cast<const f32x4*>(&Gst[b3][0][r0]);
        dc[ti] = *reinterpret_cast<const f32x4*>(&Gst[b3][1][r0]);
      }


      // X = K S on the four rho-ordered token tiles, k-block by k-block:
      // state tiles 2b, 2b+1 (rounded to fp16) feed k-block b
      f32x4 X[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) X[ti] = zero4();
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const u16x8 sh = cat8(f2h4(S[2 * b]), f2h4(S[2 * b + 1]));
        Sx[b3][vs][b][lane] = sh;   // for this chunk's Q S (output wave)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) X[ti] = mfma16h(ka[b][ti], sh, X[ti]);
      }
      // Y = V - e^G X (B fragments) and vnew = Tb Y, k-block 0 first: row
      // tiles 0 and 1 of vnew are then complete
      auto vf = [&](int ti) {
        return f32x4{bf2f(v4[ti][0]), bf2f(v4[ti][1]), bf2f(v4[ti][2]), bf2f(v4[ti][3])};
      };
      auto yfrag = [&](int b) {
        return cat8(f2h4(vf(2 * b) - eg[2 * b] * X[2 * b]),
                    f2h4(vf(2 * b + 1) - eg[2 * b + 1] * X[2 * b + 1]));
      };
      f32x4 vn[4];
      {
        const u16x8 y0 = yfrag(0);
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) vn[ti] = mfma16h(ta[tb_slot(ti, 0)], y0, zero4());
      }
      // K^T fragments of the update: element i of lane (m, grp) for state
      // tile t, k-block b is K[32 b + 8 grp + i][rho(16 t + m)], two
      // transposing reads of 4 token rows each
      u16x8 kt[2][ST];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int t = 0; t < ST; ++t) {
          const unsigned char* p = Kb + tr_off[t >> 1] + KL::RS * 32 * b + 8 * (t & 1);
          const u16x4 lo4 = lds_tr16(reinterpret_cast<const uint16_t*>(p));
          const u16x4 hi4 = lds_tr16(reinterpret_cast<const uint16_t*>(p + KL::RS * 4));
          kt[b][t] = cat8(lo4, hi4);
        }
      }
      {
        const u16x8 y1 = yfrag(1);
#pragma unroll
        for (int ti = 2; ti < 4; ++ti) vn[ti] = mfma16h(ta[tb_slot(ti, 1)], y1, vn[ti]);
      }
      // U = e^(G_last - G) vnew and vnew itself (both fp16, the latter for
      // the output waves); S = e^G_last S + K^T U, k-block by k-block
#pragma unroll
      for (int t = 0; t < ST; ++t) S[t] = S[t] * egl;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const u16x8 uh = cat8(f2h4(dc[2 * b] * vn[2 * b]), f2h4(dc[2 * b + 1] * vn[2 * b + 1]));
        Vx[b3][vs][b][lane] = cat8(f2h4(vn[2 * b]), f2h4(vn[2 * b + 1]));
#pragma unroll
        for (int t = 0; t < ST; ++t) S[t] = mfma16h(kt[b][t], uh, S[t]);
      }
      __syncthreads();   // chunk c's outputs published; stage buffer c % 3 free
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    int c = 0;
    for (; c + 2 < nc; c += 3) {
      step(I0{});
      step(I1{});
      step(I2{});
    }
    if (c < nc) step(I0{});
    if (c + 1 < nc) step(I1{});
    if (ht) {
#pragma unroll
      for (int t = 0; t < ST; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) ht[tile + (size_t)rho_row(t, 4 * grp + r) * V] = S[t][r];
      }
    }
  };
  if (w < NS) {
    if (w == 0) state_wave(std::integral_constant<int, 0>{});
    else state_wave(std::integral_constant<int, NS - 1>{});
  } else if (w == NS) {
    // ------------------------------------------------------ stage wave ----
    // Issues chunk j+2's K rows and Tb fragments straight to LDS during step
    // j (buffer_load ... lds: 16 bytes per lane, 1 KiB per instruction, lane
    // l to bytes 16 l of the block) and, before the step's barrier, waits
    // for chunk j+1's, issued during step j-1.  The wave writes LDS in no
    // other way: the compiler would wait for every load in flight before
    // such a write.  Its barriers are bare s_barriers (a workgroup release
    // fence would wait for the loads still in flight for the next step),
    // with signal fences so that no LDS access moves across them.
    typedef __attribute__((address_space(3))) void* lds_ptr;
    constexpr int kKT = (RAWK ? 0 : KL::LOADS) + 6 + 2 * NS;  // loads per stage: K, Tb, V tiles
    // chunk j's data into buffer jb % 3 (past the last chunk the loads repeat
    // it into a buffer no step reads, which keeps every step's count equal):
    // the prep kernel's fp16 K block (already in KLayout, rows past the
    // sequence end zero; not with RAWK) and Tb fragments (already in rho row
    // order), both contiguous, so lane l of load i copies bytes 16 (64 i + l)
    auto issue_kt = [&](int j, int jb) {
      const int ci = c_begin + j, buf = jb % 3;
      if constexpr (!RAWK) {
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            ws.k16 + ((size_t)ci * Hqk + hq) * KL::BYTES, 0, KL::BYTES, kBufferFlags);
#pragma unroll
        for (int i = 0; i < KL::LOADS; ++i)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr)(Kst[buf] + 1024 * i), 16,
                                                   1024 * i + 16 * lane, 0, 0, 0);
      }
      const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
          ws.tfrag + ((size_t)ci * Hv + h) * 6 * 64, 0, 6 * 64 * 16, kBufferFlags);
#pragma unroll
      for (int i = 0; i < 6; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_ptr)&Tst[buf][i][0], 16,
                                                 1024 * i + 16 * lane, 0, 0, 0);
      // V tiles: load x of slice sl, lane l copies half l % 2 of token row
      // 32 x + l / 2 (rows past the sequence end read as 0)
      const int t0 = s + j * kChunk, L = min(kChunk, e - t0);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(v + (size_t)t0 * Hv * V), 0, L * Hv * V * 2, kBufferFlags);
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
#pragma unroll
        for (int x = 0; x < 2; ++x)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rv, (lds_ptr)&Vrw[buf][sl][32 * x][0], 16,
              ((32 * x + (lane >> 1)) * Hv * V + h * V + 16 * (vt0 + sl)) * 2 + 16 * (lane & 1),
              0, 0, 0);
      }
    };
    auto barrier = [] {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };
    if (nc > 0) {
      issue_kt(0, 0);
      issue_kt(min(1, nc - 1), 1);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kKT));   // chunk 0
    }
    barrier();
    for (int j = 0; j < nc; ++j) {
      issue_kt(min(j + 2, nc - 1), j + 2);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kKT));   // chunk j+1
      barrier();
    }
  } else if (RAWK && w == NS + 2) {
    // ---------------------------------------------------- convert wave ----
    // During step j: loads chunk j+2's bf16 K rows into register set j % 2
    // (load i, lane l: 16 bytes l % (K / 8) of row (64 / (K / 8)) i + l /
    // (K / 8); rows past the sequence end read as 0), waits for chunk j+1's
    // (issued during step j-1) and writes them, as fp16, into chunk j+1's
    // KLayout block (rows past the end 0: the state update K^T U must not see
    // them); before step 0, chunk 0's.  Its LDS traffic is that block only.
    constexpr int UPR = K / 8, RPL = 64 / UPR;
    typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
    u32x4v xa[KL::LOADS], xb[KL::LOADS];
    auto load = [&](u32x4v (&x)[KL::LOADS], int c) {
      const int t0 = s + c * kChunk, L = min(kChunk, e - t0);
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(kraw + ((size_t)t0 * Hqk + hq) * K), 0, L * Hqk * K * 2,
          kBufferFlags);
#pragma unroll
      for (int i = 0; i < KL::LOADS; ++i)
        x[i] = __builtin_amdgcn_raw_buffer_load_b128(
            rk, (RPL * i + lane / UPR) * Hqk * K * 2 + 16 * (lane % UPR), 0, 0);
    };
    auto convert = [&](const u32x4v (&x)[KL::LOADS], int c) {
      const int t0 = s + c * kChunk, L = min(kChunk, e - t0);
      unsigned char* dst = Kst[c % 3];
      if (L == kChunk) {   // a whole chunk: nothing to mask
#pragma unroll
        for (int i = 0; i < KL::LOADS; ++i)
          *reinterpret_cast<u32x4v*>(dst + KL::off(RPL * i + lane / UPR, lane % UPR)) =
              __builtin_bit_cast(u32x4v, bf2h8(__builtin_bit_cast(u16x8, x[i])));
      } else {
#pragma unroll
        for (int i = 0; i < KL::LOADS; ++i) {
          const int row = RPL * i + lane / UPR, u = lane % UPR;
          const unsigned keep = row < L ? 0xFFFFFFFFu : 0u;
          *reinterpret_cast<u32x4v*>(dst + KL::off(row, u)) =
              __builtin_bit_cast(u32x4v, bf2h8(__builtin_bit_cast(u16x8, x[i]))) & keep;
        }
      }
    };
    if (nc > 0) {
      load(xa, 0);
      load(xb, min(1, nc - 1));
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(KL::LOADS));   // chunk 0
      convert(xa, 0);
    }
    __syncthreads();
    auto step = [&](int j, u32x4v (&mine)[KL::LOADS], u32x4v (&next)[KL::LOADS]) {
      load(mine, min(j + 2, nc - 1));
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(KL::LOADS));   // chunk j+1
      if (j + 1 < nc) convert(next, j + 1);
      __syncthreads();
    };
    int j = 0;
    for (; j + 1 < nc; j += 2) {
      step(j, xa, xb);
      step(j + 1, xb, xa);
    }
    if (j < nc) step(j, xa, xb);
  } else {
    // ------------------------------------------------ output / save waves ----
    // Forms with o: two output waves (below) and, with the saves too, a save
    // wave.  Forms without o (the backward's recomputation): one wave that
    // writes the gate factors and stores the saves.
    // with both outputs, the saves go to a wave of their own
    constexpr bool kSplit = SAVE && OUT;
    // SAVE: the chunk's start state (hs[chunk][v-head] = S^T, [V][K], the
    // hi fragments) and its deltas (dl, token-major); live = false stores
    // to empty resources (dropped)
    auto save_chunk = [&](int j, bool live) {
      const int t0 = s + j * kChunk, L = live ? min(kChunk, e - t0) : 0;
      const int b3 = j % 3;
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
      const int vt = vt0 + sl;
      // store i, lane l: row 16 vt + rpi i + l / cpr, columns 8 (l % cpr)
      // .. + 7, i.e. rpi whole rows per store (fragment lane r16 + 16 grp
      // of k-block b holds row r16, columns 32 b + 8 grp .. + 7); whole
      // rows measured 2 % faster than four 64-byte pieces of 16 rows
      constexpr int cpr = K / 8, rpi = 64 / cpr;
      const int c8 = lane % cpr;
      u16x8 sh[KB];
      if (live) {
#pragma unroll
        for (int i = 0; i < KB; ++i)
          sh[i] = h2bf8(Sx[b3][sl][c8 >> 2][(rpi * i + lane / cpr) + 16 * (c8 & 3)]);
      }
      const size_t ci = live ? (size_t)(c_begin + j) : 0;
      const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
          ws.hs + (ci * Hv + h) * V * K, 0, live ? V * K * 2 : 0, kBufferFlags);
#pragma unroll
      for (int i = 0; i < KB; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sh[i]), hr,
                                               ((16 * vt + rpi * i + lane / cpr) * K + 8 * c8) * 2,
                                               0, kStoreStream);
      // deltas: lane t gathers token row t (its 16 columns) from the vnew
      // fragments in LDS -- element (t % 8) of fragment lane 16 ((t / 8) % 4)
      // + n of k-block t / 32 -- and stores it into the chunk's d block
      // ([V / 8 column groups][64 tokens][8], each store one contiguous 1 KiB;
      // rows past the sequence end 0)
      const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
          ws.dl + (ci * Hv + h) * 64 * V, 0, live ? 64 * V * 2 : 0, kBufferFlags);
      u16x8 d0 = {0, 0, 0, 0, 0, 0, 0, 0}, d1 = d0;
      if (live && lane < L) {
        const uint16_t* src =
            reinterpret_cast<const uint16_t*>(&Vx[b3][sl][lane >> 5][16 * ((lane >> 3) & 3)]) +
            (lane & 7);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          d0[c] = src[8 * c];
          d1[c] = src[8 * (c + 8)];
        }
        d0 = h2bf8(d0);
        d1 = h2bf8(d1);
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, d0), dr,
                                             ((2 * vt) * 64 + lane) * 16, 0, kStoreStream);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, d1), dr,
                                             ((2 * vt + 1) * 64 + lane) * 16, 0, kStoreStream);
      }
    };
    if (kSplit && w == NS + 2) {
      // the save wave: chunk j-1's state and deltas during step j
      __syncthreads();
      for (int j = 0; j < nc; ++j) {
        if (j >= 1) save_chunk(j - 1, true);
        __syncthreads();
      }
      if (nc > 0) save_chunk(nc - 1, true);
      return;
    }
    if constexpr (OUT) {
      // ------------------------------------------- output waves (split) ----
      // Two output waves, each forming two of a chunk's four 16-row o tiles --
      // tiles 0 and 3 (role NS + 1) and tiles 1 and 2 (the last role), so that
      // each takes three P fragments and eleven MFMAs -- with the register
      // sets, step order and exact waits of the one-wave form below, over half
      // its Q rows (the caller's bf16 rows with RAWQ, else the prep's fp16
      // fragments); the first also loads G and writes the gate factors.  Each
      // wave's two tiles go out as one 16-byte store per lane.
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      auto run = [&](auto hfc) {
        constexpr int HF = decltype(hfc)::value;
        constexpr int T0 = HF ? 1 : 0, T1 = HF ? 2 : 3;
        constexpr int kQP = 2 * KB + 3;    // Q rows of two tiles, three P fragments
        constexpr int kVG = HF ? 0 : 1;    // G
        constexpr int kStores = NS;   // one o store per V tile
        constexpr int kWait = (kStores + kQP + kVG) + kStores;
        struct Regs {
          u16x8 qf[2][KB];   // Q rows 16 T + r16 (T = T0, T1), B operand of (Q S)^T
          u16x8 pf[3];       // P fragments tb_slot(T0, 0), tb_slot(T1, 0), tb_slot(T1, 1)
          float G;
        };
        Regs rA, rB;
        auto load_qp = [&](Regs& r, int j) {
          const int ci = c_begin + j;
          if constexpr (RAWQ) {
            const int t0 = s + j * kChunk, L = min(kChunk, e - t0);
            const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t*>(qraw + ((size_t)t0 * Hqk + hq) * K), 0, L * Hqk * K * 2,
                kBufferFlags);
#pragma unroll
            for (int x = 0; x < 2; ++x) {
              const int ti = x ? T1 : T0;
#pragma unroll
              for (int b = 0; b < KB; ++b)
                r.qf[x][b] = __builtin_bit_cast(
                    u16x8, __builtin_amdgcn_raw_buffer_load_b128(
                               rq, ((16 * ti + r16) * Hqk * K + 32 * b + 8 * grp) * 2, 0, 0));
            }
          } else {
            const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
                ws.q16 + ((size_t)ci * Hqk + hq) * 4 * KB * 64, 0, 4 * KB * 64 * 16, kBufferFlags);
#pragma unroll
            for (int x = 0; x < 2; ++x) {
              const int ti = x ? T1 : T0;
#pragma unroll
              for (int b = 0; b < KB; ++b)
                r.qf[x][b] = __builtin_bit_cast(
                    u16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, ((ti * KB + b) * 64 + lane) * 16,
                                                                 0, 0));
            }
          }
          const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
              ws.pfrag + ((size_t)ci * Hv + h) * 6 * 64, 0, 6 * 64 * 16, kBufferFlags);
          constexpr int slot[3] = {tb_slot(T0, 0), tb_slot(T1, 0), tb_slot(T1, 1)};
#pragma unroll
          for (int i = 0; i < 3; ++i)
            r.pf[i] = __builtin_bit_cast(
                u16x8, __builtin_amdgcn_raw_buffer_load_b128(rp, (slot[i] * 64 + lane) * 16, 0, 0));
        };
        auto load_vg = [&](Regs& r, int j) {
          const int ci = c_begin + j;
          const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
              const_cast<float*>(ws.gate + ((size_t)ci * Hv + h) * 64), 0, 256, kBufferFlags);
          r.G = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, lane * 4, 0, 0));
        };
        auto write_vg = [&](const Regs& r, int j) {
          const int buf = j % 3;
          const int t0 = s + j * kChunk, L = min(kChunk, e - t0);
          const float GL = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r.G), L - 1));
          const float eg = __expf(r.G);
          Gst[buf][0][lane] = eg;
          Gst[buf][1][lane] = __expf(GL - r.G);
          if (lane == L - 1) Egl[buf] = eg;
        };
        // o^T tiles T0, T1 of chunk j (lane (r16, grp): token row 16 T + r16,
        // columns 16 vt0 + 4 grp .. + 3)
        auto out_form = [&](const Regs& r, int j, bool live, u16x4 (&ov)[NS][2]) {
          const int b3 = j % 3;
#pragma unroll
          for (int sl = 0; sl < NS; ++sl) ov[sl][0] = ov[sl][1] = u16x4{0, 0, 0, 0};
          if (!live) return;
#pragma unroll
          for (int sl = 0; sl < NS; ++sl) {
            u16x8 sh[KB];
#pragma unroll
            for (int b = 0; b < KB; ++b) {
              sh[b] = Sx[b3][sl][b][lane];
              if constexpr (RAWQ) sh[b] = h2bf8(sh[b]);   // B of the bf16 Q S
            }
            const u16x8 vx0 = Vx[b3][sl][0][lane], vx1 = Vx[b3][sl][1][lane];
#pragma unroll
            for (int x = 0; x < 2; ++x) {
              const int ti = x ? T1 : T0;
              f32x4 qa = zero4(), qb = zero4();
#pragma unroll
              for (int b = 0; b < KB; b += 2) {
                if constexpr (RAWQ) {
                  qa = mfma16(sh[b], r.qf[x][b], qa);
                  qb = mfma16(sh[b + 1], r.qf[x][b + 1], qb);
                } else {
                  qa = mfma16h(sh[b], r.qf[x][b], qa);
                  qb = mfma16h(sh[b + 1], r.qf[x][b + 1], qb);
                }
              }
              f32x4 pv = mfma16h(vx0, r.pf[x ? 1 : 0], zero4());
              if (x == 1) pv = mfma16h(vx1, r.pf[2], pv);   // T1 >= 2: k-block 1 too
              const float egi = Gst[b3][0][16 * ti + r16];
              ov[sl][x] = f2bf4((scale * egi) * (qa + qb) + pv);
            }
          }
        };
        // v_permlane16_swap (vdst = tile T0, src = tile T1) trades rows 1, 3 of
        // vdst with rows 0, 2 of src: a lane of even grp then holds columns
        // 4 grp .. + 7 of tile T0's row, a lane of odd grp columns 4 (grp - 1)
        // .. + 7 of tile T1's row; one store per V tile
        auto out_store = [&](const u16x4 (&ov)[NS][2], int j, bool live) {
          const int t0 = s + j * kChunk, L = live ? min(kChunk, e - t0) : 0;
          const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
              o + (size_t)(live ? t0 : 0) * Hv * V, 0, L * Hv * V * 2, kBufferFlags);
#pragma unroll
          for (int sl = 0; sl < NS; ++sl) {
            const u32x2 m0 = __builtin_bit_cast(u32x2, ov[sl][0]);
            const u32x2 m1 = __builtin_bit_cast(u32x2, ov[sl][1]);
            u32x4 row;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const auto sw = __builtin_amdgcn_permlane16_swap(m0[k], m1[k], false, false);
              row[k] = sw[0];
              row[2 + k] = sw[1];
            }
            __builtin_amdgcn_raw_buffer_store_b128(
                row, orsrc,
                (((16 * ((grp & 1) ? T1 : T0) + r16) * Hv + h) * V + 16 * (vt0 + sl) +
                 4 * (grp & 2)) * 2,
                0, 0);
          }
        };
        u16x4 ov[NS][2];
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) ov[sl][0] = ov[sl][1] = u16x4{0, 0, 0, 0};
        if (nc > 0) {
          if constexpr (HF == 0) {
            load_vg(rA, 0);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            write_vg(rA, 0);
            load_vg(rB, min(1, nc - 1));
          }
          out_store(ov, 0, false);
          load_qp(rA, 0);
          if constexpr (HF == 0) load_vg(rA, min(2, nc - 1));
          out_store(ov, 0, false);
        }
        __syncthreads();
        auto step = [&](int j, Regs& r) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWait));   // chunk j-1's Q / P, chunk j+1's G
          if constexpr (HF == 0) {
            if (j + 1 < nc) write_vg(r, j + 1);
          }
          out_form(r, j - 1, j >= 1, ov);
          load_qp(r, min(j + 1, nc - 1));
          if constexpr (HF == 0) load_vg(r, min(j + 3, nc - 1));
          out_store(ov, j - 1, j >= 1);
          __syncthreads();
        };
        int j = 0;
        for (; j + 1 < nc; j += 2) {
          step(j, rB);
          step(j + 1, rA);
        }
        if (j < nc) step(j, rB);
        if (nc > 0) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
          out_form((nc - 1) & 1 ? rB : rA, nc - 1, true, ov);
          out_store(ov, nc - 1, true);
        }
      };
      if (w == chain_waves<SAVE, OUT, NS, RAWK>() - 1) run(std::integral_constant<int, 1>{});
      else run(std::integral_constant<int, 0>{});
    } else {
      // During step j: writes chunk j+1's gate factors into stage buffer
      // (j+1) % 3 and stores chunk j-1's saves (state and deltas), then loads
      // chunk j+3's G into a register set loaded two steps before it is used
      // (two sets, the loop unrolled by two); every step issues the same
      // loads and stores, so each wait names an exact count.  The stores go
      // after the step's load and the step's wait leaves the previous step's
      // stores in flight too (the counter retires loads and stores in issue
      // order): each store has two steps to drain.
      constexpr int kSave = SAVE ? NS * (KB + 2) : 0;   // state and delta stores per chunk
      constexpr int kWait = (kSave + 1) + kSave;
      struct Regs {
        float G;   // G of token `lane`
      };
      Regs rA, rB;
      auto load_vg = [&](Regs& r, int j) {
        const int ci = c_begin + j;
        const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(ws.gate + ((size_t)ci * Hv + h) * 64), 0, 256, kBufferFlags);
        r.G = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, lane * 4, 0, 0));
      };
      auto write_vg = [&](const Regs& r, int j) {
        const int buf = j % 3;
        const int t0 = s + j * kChunk, L = min(kChunk, e - t0);
        const float GL = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r.G), L - 1));
        const float eg = __expf(r.G);
        Gst[buf][0][lane] = eg;
        Gst[buf][1][lane] = __expf(GL - r.G);
        if (lane == L - 1) Egl[buf] = eg;
      };
      // the prologue issues one such group per step before step 0 (loads for
      // steps 0 and 1, stores dropped), so every wait of the loop names an
      // exact count
      if (nc > 0) {
        load_vg(rA, 0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        write_vg(rA, 0);
        load_vg(rB, min(1, nc - 1));
        if constexpr (SAVE) save_chunk(0, false);
        load_vg(rA, min(2, nc - 1));
        if constexpr (SAVE) save_chunk(0, false);
      }
      __syncthreads();
      // step j works on register set (j + 1) % 2
      auto step = [&](int j, Regs& r) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWait));   // chunk j+1's G
        if (j + 1 < nc) write_vg(r, j + 1);
        load_vg(r, min(j + 3, nc - 1));
        if constexpr (SAVE) save_chunk(j - 1, j >= 1);
        __syncthreads();
      };
      int j = 0;
      for (; j + 1 < nc; j += 2) {
        step(j, rB);
        step(j + 1, rA);
      }
      if (j < nc) step(j, rB);
      if constexpr (SAVE) {
        if (nc > 0) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
          save_chunk(nc - 1, true);
        }
      }
    }
  }
}

template <int K, bool SAVE, bool OUT>
void launch_chain_sw(const uint16_t* v, const uint16_t* qraw, const uint16_t* kraw,
                     const float* h0, float* ht, uint16_t* o, const int32_t* cu, int N, int T,
                     int total, int Hqk, int Hv, int V, float scale, const ChunkWs& ws,
                     hipStream_t st) {
  // two V tiles per workgroup once the chains fill the GPU twice over: the
  // tiles share the stage and output waves' operand traffic, and every chain
  // still has a state wave of its own (not with both outputs, where a save
  // wave would make six waves; not with RAWK, see above)
  const long long chains = (long long)N * Hv * (V / 16);
  const bool rawq = OUT && qraw;
  const bool rawk = OUT && !SAVE && rawq && kraw;
  const bool two = !(SAVE && OUT) && !rawk && chain_two_tiles(N, Hv, V);
  const dim3 grid((unsigned)(two ? chains / 2 : chains));
  auto go = [&](auto kern, int waves) {
    hipLaunchKernelGGL(kern, grid, dim3(waves * 64), 0, st, v, qraw, kraw, h0, ht, o, cu, N, T,
                       total, Hqk, Hv, V, scale, ws);
  };
  if constexpr (OUT) {
    if constexpr (!SAVE) {
      if (rawk) return go(chunk_chain_sw_kernel<K, false, true, 1, true, true>,
                          chain_waves<false, true, 1, true>());
    }
    if (rawq) {
      if (two)
        return go(chunk_chain_sw_kernel<K, SAVE, OUT, SAVE ? 1 : 2, false, true>,
                  chain_waves<SAVE, OUT, SAVE ? 1 : 2, false>());
      return go(chunk_chain_sw_kernel<K, SAVE, OUT, 1, false, true>,
                chain_waves<SAVE, OUT, 1, false>());
    }
  }
  if (two)
    go(chunk_chain_sw_kernel<K, SAVE, OUT, (SAVE && OUT) ? 1 : 2, false, false>,
       chain_waves<SAVE, OUT, (SAVE && OUT) ? 1 : 2, false>());
  else
    go(chunk_chain_sw_kernel<K, SAVE, OUT, 1, false, false>, chain_waves<SAVE, OUT, 1, false>());
}

#define GDN_CHAIN_INST(K_, SAVE_, OUT_)                                                     \
  template void launch_chain_sw<K_, SAVE_, OUT_>(                                           \
      const uint16_t*, const uint16_t*, const uint16_t*, const float*, float*, uint16_t*,   \
      const int32_t*, int, int, int, int, int, int, float, const ChunkWs&, hipStream_t);
GDN_CHAIN_INST(64, false, true)
GDN_CHAIN_INST(64, true, false)
GDN_CHAIN_INST(64, true, true)
GDN_CHAIN_INST(128, false, true)
GDN_CHAIN_INST(128, true, false)
GDN_CHAIN_INST(128, true, true)
#undef GDN_CHAIN_INST

}  // namespace gdn
