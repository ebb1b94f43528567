// Internal interface between the chunked forward (gdn_chunk.hip) and the
// chunked backward (gdn_chunk_bwd.hip): the workspace layout, sequence
// bounds, the transposing LDS read and the forward launcher the backward
// reuses to recompute (and save) the forward chain.
#pragma once

#include <atomic>

#include "gdn_common.h"

namespace gdn {

// Device workspace of one chunked call, per (global chunk, v-head) unless
// stated.  The backward-only buffers are NULL in a plain forward call.
struct ChunkWs {
  int32_t* off;     // [N+1] first global chunk of each sequence
  int32_t* status;  // [1] 0, or the cu_seqlens violation the chunk table found
  float* gate;      // [NC][Hv][64]: G_i, the chunk-local cumulative log-decay
  u16x8* tfrag;     // [NC][Hv][6 slots][64 lanes] fp16 A-operand fragments of Tb,
                    // rows in the chain's rho order, slot tb_slot(row tile, k-block)
  u16x8* pfrag;     // [NC][Hv][6][64] fp16 A-operand fragments of P, natural rows
                    // (not written by the backward's recomputation)
  unsigned char* k16;  // [NC][Hqk][KLayout<K>::BYTES] the chunk's K rows as fp16 in
                       // the chain's LDS layout (rows past the sequence end 0)
  u16x8* q16;       // [NC][Hqk][4 row tiles][K/32 k-blocks][64] fp16 B-operand
                    // fragments of the chunk's Q rows (forms that write o)
                    // (k16 / q16 NULL where the plan has no such copy: WsPlan)
  uint16_t* qn;     // l2-normalised q, k rows [B*T][Hqk][K] bf16 (use_qk_l2norm with
  uint16_t* kn;     // the backward), written by the prep kernel
  // backward only
  float* tmat;      // [NC][Hv][10][16][16] T = (I + A)^-1 (fp32): its lower 16 x 16
                    // blocks (rt, cb), cb <= rt, in the order tmat_block() gives,
                    // each row-major (the diagonal blocks' upper part 0)
  // (the three below: rows in the reverse chain's rho order, so that each
  // (tile, k-block) fragment is one contiguous 1 KiB block)
  u16x8* ttfrag;    // [NC][Hv][6][64] fp16 A-operand fragments of Tb^T, slot
                    // tb_slot(row tile, k-block)
  u16x8* ptfrag;    // [NC][Hv][4][2][64] bf16 A-operand fragments of P^T
                    // (both: row tiles 2, 3 of k-block 0 are zero, P^T's left unwritten)
  u16x8* qtfrag;    // [NC][Hqk][K/16][2][64] fp16 A-operand fragments of Q^T (key-row
                    // tile, token k-block; the l2-normalised q with use_qk_l2norm)
  uint16_t* hs;     // [NC][Hv][V][K] bf16: state at the start of every chunk, transposed
  uint16_t* dl;     // [NC][Hv][V/8][64][8] bf16: d = vnew, the per-token delta, per
                    // chunk in column groups of 8 (rows past the sequence end 0)
};

// Packed T: the 10 lower 16 x 16 blocks of the 64 x 64 matrix, block
// (rt, cb) at index rt (rt + 1) / 2 + cb; the upper blocks are zero and not
// stored.
constexpr int kTBlocks = 10;
constexpr int kTPacked = kTBlocks * 256;   // floats per (chunk, v-head)
__host__ __device__ constexpr int tmat_block(int rt, int cb) { return rt * (rt + 1) / 2 + cb; }
__host__ __device__ constexpr int tmat_block_row(int bi) {
  return bi >= 6 ? 3 : (bi >= 3 ? 2 : (bi >= 1 ? 1 : 0));
}

// Devices the library keeps per-device state for (compute-unit counts here,
// the no-allocation scratch address in gdn_chunk.hip).
constexpr int kMaxDevices = 256;

// Compute units of the current device, looked up once per device (any host
// thread may call this; the cache entries are atomic).
inline int device_cus() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int cus = cache[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

__device__ __forceinline__ void seq_bounds(const int32_t* cu, int n, int T, int total,
                                           int& s, int& e) {
  if (cu) {
    s = min(max(cu[n], 0), total);
    e = min(max(cu[n + 1], s), total);
  } else {
    s = n * T;
    e = s + T;
  }
}

// The contract on cu_seqlens [N+1]: cu[0] == 0, cu[n] <= cu[n+1], cu[N] ==
// total.  Returns 0, or the first violation found: 1 cu[0] != 0, 2 a
// decrease, 3 cu[N] != total.  The chunk table kernel checks the same three
// conditions on the device.
__host__ __device__ inline int cu_seqlens_violation(const int32_t* cu, int N, int total) {
  if (cu[0] != 0) return 1;
  for (int n = 0; n < N; ++n)
    if (cu[n + 1] < cu[n]) return 2;
  return cu[N] != total ? 3 : 0;
}

// Buffers zero-filled when the chunk table found a cu_seqlens violation.
struct ZeroList {
  void* p[5];
  size_t bytes[5];
};

// Enqueue the zero-fill of `z` conditional on *status != 0 (one small launch;
// its workgroups return at once when the status is 0).
void launch_zero_on_violation(const int32_t* status, const ZeroList& z, hipStream_t st);

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// (i % 4) of the 4 x 16-bit words read by lanes 4m + i / 4, m = 0..3.  A
// group reading 4 rows x 16 columns of a row-major tile thus gets the tile's
// columns: lane i holds column i of the 4 rows.
__device__ __forceinline__ u16x4 lds_tr16(const uint16_t* p) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (s16x4 __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(u16x4, r);
}

// A-operand fragment of X^T (equivalently the B-operand fragment of X) from
// a row-major bf16 tile X in LDS with row stride ld: lane (r16, grp) gets
// X[k0 + 8 grp + i][m0 + r16], i = 0..7.  m0 % 4 == 0 and ld % 4 == 0.
__device__ __forceinline__ u16x8 lds_colfrag(const uint16_t* X, int ld, int k0, int m0,
                                             int lane) {
  const int r16 = lane % 16, grp = lane / 16;
  const int m4 = r16 >> 2, q4 = r16 & 3;
  const u16x4 lo = lds_tr16(X + (k0 + 8 * grp + m4) * ld + m0 + 4 * q4);
  const u16x4 hi = lds_tr16(X + (k0 + 8 * grp + 4 + m4) * ld + m0 + 4 * q4);
  return u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// ------------------------------------------- state-wave chain helpers ----
// (the forward chain gdn_chunk_chain.hip and the reverse chain
// gdn_chunk_rev.hip)

// rho of tile row 16 T + m (m < 16)
__device__ __forceinline__ int rho_row(int T, int m) {
  return 32 * (T >> 1) + 8 * (m >> 2) + 4 * (T & 1) + (m & 3);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u16x8 cat8(u16x4 a, u16x4 b) {
  return u16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Tb / P fragment slot of (row tile ti, k-block b): row tiles 0 and 1 have
// no k-block 1 (both are lower triangular), so six slots.
__device__ __forceinline__ constexpr int tb_slot(int ti, int b) { return b == 0 ? ti : 2 + ti; }

// s_waitcnt immediate (gfx9 encoding) that waits until at most n
// vector-memory operations are outstanding, and for nothing else.
__device__ __forceinline__ constexpr int vmcnt_imm(int n) {
  return 0x0F70 | (n & 15) | (((n >> 4) & 3) << 14);
}

// Staged K rows: 2K bytes per row, unpadded, the row's 16-byte units
// (8 keys each) permuted by XOR with swz(row), which takes row bits 3-4 to
// unit bits 0-1 and row bits 0-1 (K = 128; bit 1 for K = 64) to the unit
// bits above.  Both fragment reads of the state wave then fall on distinct
// banks across each 16 lanes: the column-fragment reads (16 rows rho(16 ti
// + m), one unit) and the transposing reads (4 rows x 4 units); row bits 2
// and 5 do not enter swz, so every K read is one of a few per-lane bases
// plus a compile-time offset.
template <int K>
struct KLayout {
  static constexpr int RS = 2 * K;                 // row stride (bytes)
  static constexpr int BYTES = 64 * RS;            // buffer size
  static constexpr int LOADS = BYTES / 1024;       // 1 KiB direct-to-LDS loads
  __device__ static constexpr int swz(int r) {
    return ((r >> 3) & 3) | ((K == 128 ? (r & 3) : ((r >> 1) & 1)) << 2);
  }
  // byte offset of unit u (keys 8u .. 8u + 7) of row r
  __device__ static constexpr int off(int r, int u) { return r * RS + 16 * (u ^ swz(r)); }
};

// Whether a chunked call's forward chain reads K from the caller's bf16 rows
// (a convert wave, one V tile per workgroup) rather than the prep kernel's
// fp16 copy: a forward without use_qk_l2norm whose chains do not fill the
// GPU twice over (the backward's reverse chain reads the copy, and two V
// tiles per workgroup leave no registers for the convert wave).  Q is read
// from the caller's rows whenever use_qk_l2norm is off.
inline bool chain_two_tiles(int N, int Hv, int V) {
  return V % 32 == 0 && (long long)N * Hv * (V / 16) >= 2LL * device_cus();
}
inline bool chain_reads_rows(bool bwd, bool l2, int N, int Hv, int V) {
  return !bwd && !l2 && !chain_two_tiles(N, Hv, V);
}

// Workspace plan (byte offsets into the caller's buffer).
struct WsPlan {
  size_t off, status, gate, tfrag, pfrag, k16, q16, qn, kn, total;
  bool k16_copy, q16_copy;   // k16 / q16 planned (else the chains read the caller's rows)
  // backward only (0 when not planned)
  size_t tmat, ttfrag, ptfrag, qtfrag, hs, dl, dse, dd;
  long long ncmax;
};

WsPlan plan_ws(int B, int T, int Hqk, int Hv, int K, int V, int N, bool has_cu, bool l2,
               bool bwd);

// What a forward launch sequence writes: kForward = o / ht only; kRecompute =
// the backward's inputs only (prep adds tmat / ttfrag / ptfrag, the chain
// saves hs / dl; o and ht are ignored); kSave = both (a training forward).
enum class FwdMode { kForward, kRecompute, kSave };

// Enqueue the chunk table, the prep and the forward chain.
void launch_chunk_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                      const float* beta, const float* h0, float* ht, uint16_t* o,
                      const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N,
                      float scale, bool l2, FwdMode mode, const WsPlan& p, unsigned char* wsb,
                      hipStream_t st, const GateIn& gate = GateIn{});

ChunkWs ws_pointers(const WsPlan& p, unsigned char* wsb);

// Forward chain, state-wave form (gdn_chunk_chain.hip).  SAVE: the state at
// every chunk start and the per-token deltas for the backward; OUT: o, ht.
// qraw, kraw (a forward, OUT without SAVE, both non-null): K and Q from the
// caller's bf16 rows instead of ws.k16 / ws.q16.
template <int K, bool SAVE, bool OUT>
void launch_chain_sw(const uint16_t* v, const uint16_t* qraw, const uint16_t* kraw,
                     const float* h0, float* ht, uint16_t* o, const int32_t* cu, int N, int T,
                     int total, int Hqk, int Hv, int V, float scale, const ChunkWs& ws,
                     hipStream_t st);

// Reverse chain of the backward (gdn_chunk_rev.hip): dS' of every chunk into
// dse, dd into dd, dh0 (K rows from ws.k16).
template <int K>
void launch_rev_sw(const uint16_t* dO, const float* dht, float* dh0,
                   const int32_t* cu, int N, int T, int total, int Hqk, int Hv, int V,
                   float scale, const ChunkWs& ws, uint16_t* dse, uint16_t* dd, hipStream_t st);


}  // namespace gdn
