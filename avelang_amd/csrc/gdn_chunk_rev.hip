// Reverse chain of the chunked backward, state-wave form (gfx950).
//
// Per chunk, from the last to the first (dS' = dL/d(state at the chunk's
// end), c' = scale; the backward's derivation is in gdn_chunk_bwd.hip):
//     dd = P^T dO + e^(G_L - G) (K dS'),   Z = Tb^T dd,
//     dS = e^G_L dS' - K^T (e^G Z) + Q^T (c' e^G dO)
// and dS becomes the previous chunk's dS'.  Stored for the gradient kernel:
// dS' of every chunk (bf16, transposed) and dd (bf16, per chunk in column
// groups of 8); dh0.
//
// The layout of the forward chain (gdn_chunk_chain.hip), with three helper
// waves in place of its output wave:
//
//   wave 0, the state wave, holds every key row of the tile's dS' in VGPRs
//   (rho row order) and runs the dS'-dependent products alone: K dS',
//   Tb^T dd and K^T U, each one v_mfma_f32_16x16x32_f16 pass with fp16
//   operands rounded from fp32 (as the forward chain), every operand from
//   LDS and every result tile the next product's B operand where it stands.
//   The terms that do not depend on dS' -- P^T dO and Q^T (c' e^G dO) -- it
//   reads as fp32 tiles in its own layout.
//
//   wave 1, the stage wave, copies the chunk's fp16 K block and Tb^T
//   fragments two steps ahead straight into LDS (buffer_load ... lds), both
//   contiguous as the prep kernel laid them out, and the dO tile three steps
//   ahead.
//
//   waves 2 to 4, the helper waves, form the next step's gate factors and
//   P^T dO (wave 2) and Q^T (c' e^G dO) (waves 3 and 4, half the state
//   tiles each) from the prep's P^T and Q^T fragments and dO (the stage
//   wave's tile, read transposed), and write them into LDS; wave 4 also
//   stores the previous step's dS' and dd.
//
// Step j works on chunk nc - 1 - j of the sequence.
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

template <int K>
__global__ __launch_bounds__(320) void chunk_rev_sw_kernel(
    const uint16_t* __restrict__ dO, const float* dht,
    float* dh0, const int32_t* __restrict__ cu, int N, int T, int total, int Hqk, int Hv, int V,
    float scale, ChunkWs ws, uint16_t* __restrict__ dse, uint16_t* __restrict__ ddo) {
  constexpr int KB = K / 32;   // k-blocks over the key index
  constexpr int ST = K / 16;   // 16-row state tiles
  using KL = KLayout<K>;
  // stage buffers (step j in buffer j % 3): fp16 K rows (KLayout), Tb^T
  // fragments (rho rows)
  __shared__ __attribute__((aligned(16))) unsigned char Kst[3][KL::BYTES];
  __shared__ __attribute__((aligned(16))) u16x8 Tst[3][6][64];
  // helper -> state: e^G and e^(G_last - G) by token, e^G_last, P^T dO
  // (token tiles in the state wave's layout) and Q^T (c' e^G dO) (state tiles)
  __shared__ __attribute__((aligned(16))) float Gst[3][2][64];
  __shared__ float Egl[3];
  __shared__ __attribute__((aligned(16))) f32x4 Pst[3][4][64];
  __shared__ __attribute__((aligned(16))) f32x4 Qst[3][ST][64];
  // state -> helper: dS' (bf16) B fragments at the step's start, dd (bf16)
  // as B fragments
  __shared__ __attribute__((aligned(16))) u16x8 Sx[3][KB][64];
  __shared__ __attribute__((aligned(16))) u16x8 Vx[3][2][64];
  // the dO tile of step j (bf16 [token][16 columns]) in slot j % 4, copied
  // by the stage wave three steps ahead and read transposed by the helpers
  __shared__ __attribute__((aligned(16))) uint16_t Dst[4][64][16];
  __shared__ __attribute__((aligned(16))) float Eq[2][64];   // Q waves 3, 4: c' e^G by token

  const int NVT = V / 16;
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  const int unit = NVT * (Hv / Hqk);
  if (nb % (8 * unit) == 0) {
    const int i = bid >> 3;
    bid = ((i / unit) * 8 + (bid & 7)) * unit + i % unit;
  } else if ((nb & 7) == 0) {
    bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  }
  const int vt = bid % NVT;
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

  if (w == 0) {
    // ------------------------------------------------------ state wave ----
    const size_t tile = ((size_t)n * Hv + h) * (size_t)K * V + 16 * vt + r16;
    f32x4 S[ST];
    if (dht) {
#pragma unroll
      for (int t = 0; t < ST; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) S[t][r] = dht[tile + (size_t)rho_row(t, 4 * grp + r) * V];
      }
    } else {
#pragma unroll
      for (int t = 0; t < ST; ++t) S[t] = zero4();
    }
    __syncthreads();   // stage buffer 0 and step 0's dO are in
    __syncthreads();   // the helpers' step-0 tiles are in

    const int m4 = r16 >> 2, q4 = r16 & 3;
    int ka_off[KB], tr_off[ST / 2];
#pragma unroll
    for (int b = 0; b < KB; ++b) ka_off[b] = KL::off(rho_row(0, r16), 4 * b + grp);
#pragma unroll
    for (int u = 0; u < ST / 2; ++u) tr_off[u] = KL::off(8 * grp + m4, 4 * u + q4);

    auto step = [&](auto b3c) {
      constexpr int b3 = decltype(b3c)::value;
      const unsigned char* Kb = Kst[b3];
      // operands of the step, all from LDS and issued first, in the order
      // they are used
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
      f32x4 eg[4], dc[4], pd[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int r0 = 32 * (ti >> 1) + 8 * grp + 4 * (ti & 1);
        eg[ti] = *reinterpret_cast<const f32x4*>(&Gst[b3][0][r0]);
        dc[ti] = *reinterpret_cast<const f32x4*>(&Gst[b3][1][r0]);
        pd[ti] = Pst[b3][ti][lane];
      }

      // X = K dS' on the rho-ordered token tiles: state tiles 2b, 2b+1
      // (rounded to fp16) feed k-block b; dS' as bf16 to the helper's save
      f32x4 X[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) X[ti] = zero4();
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const u16x8 sh = cat8(f2h4(S[2 * b]), f2h4(S[2 * b + 1]));
        Sx[b3][b][lane] = cat8(f2bf4(S[2 * b]), f2bf4(S[2 * b + 1]));
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) X[ti] = mfma16h(ka[b][ti], sh, X[ti]);
      }
      // dd = P^T dO + e^(G_L - G) X on token tiles 2b, 2b + 1: the fp16 B
      // fragment of k-block b of Tb^T dd, and dd (bf16) for the save
      auto ddfrag = [&](int b) {
        const f32x4 d0 = pd[2 * b] + dc[2 * b] * X[2 * b];
        const f32x4 d1 = pd[2 * b + 1] + dc[2 * b + 1] * X[2 * b + 1];
        Vx[b3][b][lane] = cat8(f2bf4(d0), f2bf4(d1));
        return cat8(f2h4(d0), f2h4(d1));
      };
      // Z = Tb^T dd: Tb^T is upper triangular, so token tiles 2 and 3 have
      // no k-block 0; k-block 1 first, where every tile has a term
      f32x4 z[4];
      {
        const u16x8 y1 = ddfrag(1);
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) z[ti] = mfma16h(ta[tb_slot(ti, 1)], y1, zero4());
      }
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
        const u16x8 y0 = ddfrag(0);
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) z[ti] = mfma16h(ta[tb_slot(ti, 0)], y0, z[ti]);
      }
      // dS = e^G_L dS' + Q^T (c' e^G dO) + K^T U,  U = -e^G Z, block by block
#pragma unroll
      for (int t = 0; t < ST; ++t) S[t] = S[t] * egl + Qst[b3][t][lane];
#pragma unroll
      for (int b = 1; b >= 0; --b) {
        const u16x8 uh = cat8(f2h4(-(eg[2 * b] * z[2 * b])), f2h4(-(eg[2 * b + 1] * z[2 * b + 1])));
#pragma unroll
        for (int t = 0; t < ST; ++t) S[t] = mfma16h(kt[b][t], uh, S[t]);
      }
      __syncthreads();   // step j's outputs published; stage buffer j % 3 free
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    int j = 0;
    for (; j + 2 < nc; j += 3) {
      step(I0{});
      step(I1{});
      step(I2{});
    }
    if (j < nc) step(I0{});
    if (j + 1 < nc) step(I1{});
    if (dh0) {
#pragma unroll
      for (int t = 0; t < ST; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) dh0[tile + (size_t)rho_row(t, 4 * grp + r) * V] = S[t][r];
      }
    }
  } else if (w == 1) {
    // ------------------------------------------------------ stage wave ----
    // As in the forward chain: step j + 2's fp16 K block (KLayout, rows
    // past the sequence end zero) and Tb^T fragments (rho rows) straight to
    // LDS during step j, lane l of load i copying bytes 16 (64 i + l) of the
    // contiguous source; bare barriers, explicit waits.  With them, step
    // j + 3's dO tile (the helpers form step j + 1's terms during step j, so
    // their dO must be in one step earlier than the stage buffers).
    typedef __attribute__((address_space(3))) void* lds_ptr;
    constexpr int kKT = KL::LOADS + 6 + 2;
    const int rowd = Hv * V * 2;
    // step jd's dO tile into slot jd % 4 (past the last step: the last
    // step's again, into a slot no later step reads): load x, lane l copies
    // half l % 2 of token row 32 x + l / 2 (rows past the sequence end 0)
    auto issue_do = [&](int jd) {
      const int jc = nc - 1 - min(jd, nc - 1);
      const int t0 = s + jc * kChunk, L = min(kChunk, e - t0);
      const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(dO + (size_t)t0 * Hv * V), 0, L * rowd, kBufferFlags);
#pragma unroll
      for (int x = 0; x < 2; ++x)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rd, (lds_ptr)&Dst[jd % 4][32 * x][0], 16,
            (32 * x + (lane >> 1)) * rowd + (h * V + 16 * vt) * 2 + 16 * (lane & 1), 0, 0, 0);
    };
    auto issue_kt = [&](int j, int jb) {
      issue_do(jb + 1);
      const int ci = c_begin + nc - 1 - j, buf = jb % 3;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          ws.k16 + ((size_t)ci * Hqk + hq) * KL::BYTES, 0, KL::BYTES, kBufferFlags);
#pragma unroll
      for (int i = 0; i < KL::LOADS; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr)(Kst[buf] + 1024 * i), 16,
                                                 1024 * i + 16 * lane, 0, 0, 0);
      const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
          ws.ttfrag + ((size_t)ci * Hv + h) * 6 * 64, 0, 6 * 64 * 16, kBufferFlags);
#pragma unroll
      for (int i = 0; i < 6; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_ptr)&Tst[buf][i][0], 16,
                                                 1024 * i + 16 * lane, 0, 0, 0);
    };
    auto barrier = [] {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };
    if (nc > 0) {
      issue_do(0);
      issue_kt(0, 0);
      issue_kt(min(1, nc - 1), 1);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kKT));   // step 0's (and dO of 0, 1)
    }
    barrier();
    barrier();   // the helpers' step-0 tiles
    for (int j = 0; j < nc; ++j) {
      issue_kt(min(j + 2, nc - 1), j + 2);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kKT));   // step j+1's
      barrier();
    }
  } else {
    // ---------------------------------------------------- helper waves ----
    // Wave 2 forms step j+1's gate factors and P^T dO into LDS; waves 3 and
    // 4 form step j+1's Q^T (c' e^G dO), state tiles [0, ST/2) and [ST/2,
    // ST), and wave 4 also stores step j-1's dS' and dd (their LDS buffers
    // live until step j+2 overwrites them).  Each uses the register set it
    // loaded two steps before and then loads step j+3's operands into it.
    // Every step issues the same loads and stores, so each wait names an
    // exact count; one code path per role (a compile-time value), so that no
    // join of two roles' loads blurs the compiler's wait counts.
    typedef unsigned int u32x4l __attribute__((ext_vector_type(4)));
    // step j's dS' (dse[chunk][v-head] = dS'^T, [V][K], bf16) and dd; live =
    // false (no step yet) stores to empty resources
    auto save = [&](int j, bool live) {
      const int jc = nc - 1 - j;
      const int t0 = s + jc * kChunk, L = live ? min(kChunk, e - t0) : 0;
      const int b3 = j % 3;
      const size_t ci = live ? (size_t)(c_begin + jc) : 0;
      // store i, lane l: row 16 vt + rpi i + l / cpr, columns 8 (l % cpr)
      // .. + 7, i.e. rpi whole rows per store (fragment lane r16 + 16 grp
      // of k-block b holds row r16, columns 32 b + 8 grp .. + 7)
      constexpr int cpr = K / 8, rpi = 64 / cpr;
      const int c8 = lane % cpr;
      u16x8 sh[KB];
      if (live) {
#pragma unroll
        for (int i = 0; i < KB; ++i) sh[i] = Sx[b3][c8 >> 2][(rpi * i + lane / cpr) + 16 * (c8 & 3)];
      }
      const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
          dse + (ci * Hv + h) * V * K, 0, live ? V * K * 2 : 0, kBufferFlags);
#pragma unroll
      for (int i = 0; i < KB; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4l, sh[i]), hr,
                                               ((16 * vt + rpi * i + lane / cpr) * K + 8 * c8) * 2,
                                               0, kStoreStream);
      // lane t gathers token row t of dd from the fragments in LDS (element
      // t % 8 of fragment lane 16 ((t / 8) % 4) + n of k-block t / 32) and
      // stores it into the chunk's dd block ([V / 8 column groups][64 tokens]
      // [8], so that each store is one contiguous 1 KiB; rows past the
      // sequence end 0)
      const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
          ddo + (ci * Hv + h) * 64 * V, 0, live ? 64 * V * 2 : 0, kBufferFlags);
      u16x8 d0 = {0, 0, 0, 0, 0, 0, 0, 0}, d1 = d0;
      if (live && lane < L) {
        const uint16_t* src =
            reinterpret_cast<const uint16_t*>(&Vx[b3][lane >> 5][16 * ((lane >> 3) & 3)]) +
            (lane & 7);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          d0[c] = src[8 * c];
          d1[c] = src[8 * (c + 8)];
        }
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4l, d0), dr,
                                             ((2 * vt) * 64 + lane) * 16, 0, kStoreStream);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4l, d1), dr,
                                             ((2 * vt + 1) * 64 + lane) * 16, 0, kStoreStream);
    };
    auto helper = [&](auto rolec) {
      constexpr int role = decltype(rolec)::value;
      constexpr int QT = ST / 2;                 // Q^T state tiles per Q wave
      constexpr int t_lo = role == 2 ? QT : 0;   // this Q wave's first tile
      constexpr int kStep = role == 0 ? 6 + 1 : 2 * QT + 1 + (role == 2 ? KB + 2 : 0);
      struct Regs {
        u16x8 pt[6];        // P^T fragments (rho rows, bf16) by tb_slot (wave 2)
        u16x8 qt[QT][2];    // Q^T fragments (rho key rows, fp16) by token k-block
        float G;            // G of token `lane`
      };
      Regs rA, rB;
      auto load = [&](Regs& r, int j) {
        const int ci = c_begin + nc - 1 - j;
        if constexpr (role != 0) {
          const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
              ws.qtfrag + ((size_t)ci * Hqk + hq) * ST * 128, 0, ST * 128 * 16, kBufferFlags);
#pragma unroll
          for (int t = 0; t < QT; ++t) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
              r.qt[t][b] = __builtin_bit_cast(
                  u16x8, __builtin_amdgcn_raw_buffer_load_b128(
                             rq, ((2 * (t_lo + t) + b) * 64 + lane) * 16, 0, 0));
          }
        } else {
          const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
              ws.ptfrag + ((size_t)ci * Hv + h) * 4 * 128, 0, 4 * 128 * 16, kBufferFlags);
#pragma unroll
          for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              if (b == 0 && ti >= 2) continue;
              r.pt[tb_slot(ti, b)] = __builtin_bit_cast(
                  u16x8, __builtin_amdgcn_raw_buffer_load_b128(rp, ((2 * ti + b) * 64 + lane) * 16, 0, 0));
            }
          }
        }
        const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
            ws.gate + ((size_t)ci * Hv + h) * 64, 0, 256, kBufferFlags);
        r.G = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, lane * 4, 0, 0));
      };
      // step j's gate factors and P^T dO (wave 2) or Q^T (c' e^G dO) (waves
      // 3, 4) into buffer j % 3
      auto publish = [&](const Regs& r, int j) {
        const int buf = j % 3;
        const float eg = __expf(r.G);
        // dO B fragments: element i of lane (r16, grp), k-block kb is
        // dO[32 kb + 8 grp + i][16 vt + r16] (the stage wave's tile)
        u16x8 dof[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) dof[kb] = lds_colfrag(&Dst[j % 4][0][0], 16, 32 * kb, 0, lane);
        if constexpr (role != 0) {
          // c' e^G dO for this lane's k-slots (tokens 32 kb + 8 grp + i), fp16;
          // c' e^G of the tokens through this wave's own LDS row (written and
          // read back by the one wave, in order)
          float* eq = Eq[role - 1];
          eq[lane] = scale * eg;
          u16x8 oh[2];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            const f32x4 e0 = *reinterpret_cast<const f32x4*>(&eq[32 * kb + 8 * grp]);
            const f32x4 e1 = *reinterpret_cast<const f32x4*>(&eq[32 * kb + 8 * grp + 4]);
            f32x4 x0, x1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              x0[i] = e0[i] * bf2f(dof[kb][i]);
              x1[i] = e1[i] * bf2f(dof[kb][4 + i]);
            }
            oh[kb] = cat8(f2h4(x0), f2h4(x1));
          }
#pragma unroll
          for (int t = 0; t < QT; ++t) {
            f32x4 a = zero4();
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) a = mfma16h(r.qt[t][kb], oh[kb], a);
            Qst[buf][t_lo + t][lane] = a;
          }
        } else {
          const int jc = nc - 1 - j;
          const int t0 = s + jc * kChunk, L = min(kChunk, e - t0);
          const float GL = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r.G), L - 1));
          Gst[buf][0][lane] = eg;
          Gst[buf][1][lane] = __expf(GL - r.G);
          if (lane == L - 1) Egl[buf] = eg;
#pragma unroll
          for (int ti = 0; ti < 4; ++ti) {
            f32x4 pd = mfma16(r.pt[tb_slot(ti, 1)], dof[1], zero4());
            if (ti < 2) pd = mfma16(r.pt[tb_slot(ti, 0)], dof[0], pd);
            Pst[buf][ti][lane] = pd;
          }
        }
      };
      if (nc > 0) load(rA, 0);
      __syncthreads();   // step 0's dO is in
      if (nc > 0) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        publish(rA, 0);
        load(rB, min(1, nc - 1));
        if constexpr (role == 2) save(0, false);   // the stores a step issues, dropped
        load(rA, min(2, nc - 1));
      }
      __syncthreads();
      // step j works on register set (j + 1) % 2
      auto hstep = [&](int j, Regs& r) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kStep));   // step j+1's operands
        if (j + 1 < nc) publish(r, j + 1);
        if constexpr (role == 2) save(j - 1, j >= 1);
        load(r, min(j + 3, nc - 1));
        __syncthreads();
      };
      int j = 0;
      for (; j + 1 < nc; j += 2) {
        hstep(j, rB);
        hstep(j + 1, rA);
      }
      if (j < nc) hstep(j, rB);
      if constexpr (role == 2) {
        if (nc > 0) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
          save(nc - 1, true);
        }
      }
    };
    if (w == 2) helper(std::integral_constant<int, 0>{});
    else if (w == 3) helper(std::integral_constant<int, 1>{});
    else helper(std::integral_constant<int, 2>{});
  }
}

template <int K>
void launch_rev_sw(const uint16_t* dO, const float* dht, float* dh0, const int32_t* cu, int N,
                   int T, int total, int Hqk, int Hv, int V, float scale, const ChunkWs& ws,
                   uint16_t* dse, uint16_t* dd, hipStream_t st) {
  hipLaunchKernelGGL((chunk_rev_sw_kernel<K>), dim3(N * Hv * (V / 16)), dim3(320), 0, st, dO,
                     dht, dh0, cu, N, T, total, Hqk, Hv, V, scale, ws, dse, dd);
}

template void launch_rev_sw<64>(const uint16_t*, const float*, float*, const int32_t*, int, int,
                                int, int, int, int, float, const ChunkWs&, uint16_t*, uint16_t*,
                                hipStream_t);
template void launch_rev_sw<128>(const uint16_t*, const float*, float*, const int32_t*, int, int,
                                 int, int, int, int, float, const ChunkWs&, uint16_t*, uint16_t*,
                                 hipStream_t);

}  // namespace gdn
