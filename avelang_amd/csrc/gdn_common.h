// Shared device helpers for the gfx950 GDN kernels: bf16 packing, the
// 16x16x32 bf16 MFMA wrapper, and the thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/gdn.h"
#include "../../include/gdn_layer.h"

namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;  // tokens per chunk of the prefill path
// Word 3 of a raw (stride 0) buffer resource on gfx950: out-of-range loads
// return 0 and out-of-range stores are dropped.
constexpr int kBufferFlags = 0x00020000;
// Cache-policy operand of a buffer store for data no kernel of the same call
// reads back soon (o, the training saves, the reverse chain's dS' / dd):
// the nt (non-temporal, streaming) bit.  Whole 16-byte lanes only -- 2-byte
// stores with it measured far slower.
constexpr int kStoreStream = 2;
constexpr int kWave = 64;   // CDNA wavefront width
// s_waitcnt immediate (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8) that waits for every vector-memory load and nothing else.
constexpr int kWaitVmcnt0 = 0x0F70;

// bf16 <-> fp32 on raw 16-bit patterns.
__device__ __forceinline__ float bf2f(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// fp32 -> bf16, round to nearest even: one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Split x into hi + lo bf16 parts with x ~= hi + lo to ~2^-17 relative.
__device__ __forceinline__ void split_bf(float x, uint16_t& hi, uint16_t& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}

// Four values at once (two v_cvt_pk_bf16_f32 per conversion, and the hi
// part re-expanded from the packed words with a shift / mask): the same
// results as f2bf / split_bf per element, in fewer instructions.
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2p __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x4 f2bf4(f32x4 x) {
  return __builtin_bit_cast(u16x4, __builtin_convertvector(x, bf16x4));
}
__device__ __forceinline__ void split_bf4(f32x4 x, u16x4& hi, u16x4& lo) {
  const u32x2p hp = __builtin_bit_cast(u32x2p, __builtin_convertvector(x, bf16x4));
  const f32x4 hf = {__uint_as_float(hp[0] << 16), __uint_as_float(hp[0] & 0xffff0000u),
                    __uint_as_float(hp[1] << 16), __uint_as_float(hp[1] & 0xffff0000u)};
  hi = __builtin_bit_cast(u16x4, hp);
  lo = f2bf4(x - hf);
}

__device__ __forceinline__ bf16x8 as_bf(u16x8 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// D += A(16x32) * B(32x16), bf16 operands, fp32 accumulate.
// Operand slot (lane l, element i) carries reduction index kappa(l/16, i);
// A and B must use the same kappa.  Output: lane l holds D[4*(l/16)+r][l%16].
__device__ __forceinline__ f32x4 mfma16(u16x8 a, u16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(a), as_bf(b), c, 0, 0, 0);
}

// fp16 forms (the prefill chain's state products): fp32 -> fp16 rounds to
// nearest even, two values per v_cvt_pk_f16_f32 on gfx950.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ u16x4 f2h4(f32x4 x) {
  return __builtin_bit_cast(u16x4, __builtin_convertvector(x, f16x4));
}
// eight bf16 values as fp16 (exact for |x| in fp16's normal range)
__device__ __forceinline__ u16x8 bf2h8(u16x8 x) {
  const f32x8 f = __builtin_convertvector(__builtin_bit_cast(bf16x8, x), f32x8);
  return __builtin_bit_cast(u16x8, __builtin_convertvector(f, f16x8));
}
// eight fp16 values re-rounded to bf16 (for the backward's bf16 saves)
__device__ __forceinline__ u16x8 h2bf8(u16x8 x) {
  const f32x8 f = __builtin_convertvector(__builtin_bit_cast(f16x8, x), f32x8);
  return __builtin_bit_cast(u16x8, __builtin_convertvector(f, bf16x8));
}

// D += A(16x32) * B(32x16), fp16 operands, fp32 accumulate (same fragment
// layouts as mfma16).
__device__ __forceinline__ f32x4 mfma16h(u16x8 a, u16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// D = A B + C for fp32 16x16x4 (one block): lane l holds A[l % 16][l / 16]
// and B[l / 16][l % 16]; D has the same layout as the 16x16x32 bf16 form.
__device__ __forceinline__ f32x4 mfma4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// ------------------------------------------------------------ elements ----
template <int DT>
struct Elt;
template <>
struct Elt<GDN_DTYPE_F32> {
  using T = float;
  static constexpr int VEC = 4;
  static __device__ __forceinline__ float to_f(T v) { return v; }
  static __device__ __forceinline__ T from_f(float f) { return f; }
};
template <>
struct Elt<GDN_DTYPE_BF16> {
  using T = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f(T v) { return bf2f(v); }
  static __device__ __forceinline__ T from_f(float f) { return f2bf(f); }
};
template <>
struct Elt<GDN_DTYPE_F16> {
  using T = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f(T v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
  static __device__ __forceinline__ T from_f(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

template <int DT>
__device__ __forceinline__ float lde(const void* p, long long i) {
  return Elt<DT>::to_f(static_cast<const typename Elt<DT>::T*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void ste(void* p, long long i, float v) {
  static_cast<typename Elt<DT>::T*>(p)[i] = Elt<DT>::from_f(v);
}
// value rounded through the element type (identity for fp32)
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  return Elt<DT>::to_f(Elt<DT>::from_f(v));
}

// Load of a small parameter tensor whose element type is a runtime code.
__device__ __forceinline__ float ldp(const void* p, long long i, int dt) {
  if (dt == GDN_DTYPE_F32) return static_cast<const float*>(p)[i];
  if (dt == GDN_DTYPE_BF16) return lde<GDN_DTYPE_BF16>(p, i);
  return lde<GDN_DTYPE_F16>(p, i);
}


inline bool dtype_ok(int dt) {
  return dt == GDN_DTYPE_F32 || dt == GDN_DTYPE_BF16 || dt == GDN_DTYPE_F16;
}

// Qwen3-Next gating (modeling_qwen3_next.py:650-652) of element i (token-major
// [.., H]) of v-head h:  g = -exp(A_log[h]) * softplus(a[i] + dt_bias[h]),
// beta = sigmoid(b[i]); softplus with beta spb and threshold spt as
// torch.nn.functional.softplus.  One definition for the standalone gating
// kernel and for the core kernels that compute g and beta themselves, so
// that both paths give the same bits.
struct GateIn {
  const void* A_log;     // [H], element type pdt
  const void* a;         // [.., H], adt   (NULL: the kernel reads g / beta)
  const void* b;         // [.., H], bdt   (NULL: beta is not formed)
  const void* dt_bias;   // [H], pdt
  int adt, bdt, pdt;
  float spb, spt;
  long long n;           // elements of a, b (bounds of the flat loads)
  int H;                 // elements of A_log, dt_bias
};

// Element i of an [n] tensor of runtime element type dt, without control
// flow: a bounded 16-bit and a bounded 32-bit buffer load are both issued
// and the one the type calls for is selected (the other reads garbage or,
// past the end, 0).  The same value as ldp; a kernel that keeps loads in
// flight across this one needs it, since a branch here would make the wait
// at the join cover every outstanding load.
// The two raw words (issued now) and the value they give (formed later):
// a kernel can load early and select when the value is needed.
struct FlatRaw {
  uint16_t h;
  uint32_t w;
};
__device__ __forceinline__ FlatRaw ldp_flat_raw(const void* p, long long i, int dt, long long n) {
  const int es = dt == GDN_DTYPE_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(p), 0, p ? static_cast<int>(n * es) : 0, kBufferFlags);
  FlatRaw x;
  x.h = __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(i * 2), 0, 0);
  x.w = __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(i * 4), 0, 0);
  return x;
}
__device__ __forceinline__ float flat_value(FlatRaw x, int dt) {
  const float hf = static_cast<float>(__builtin_bit_cast(_Float16, x.h));
  return dt == GDN_DTYPE_F32 ? __uint_as_float(x.w) : (dt == GDN_DTYPE_BF16 ? bf2f(x.h) : hf);
}
__device__ __forceinline__ float ldp_flat(const void* p, long long i, int dt, long long n) {
  return flat_value(ldp_flat_raw(p, i, dt, n), dt);
}

// The per-head part (-exp(A_log[h]), dt_bias[h]) and the per-element part,
// separable so that a kernel walking many tokens of one head forms the
// first once.  FLAT: loads by ldp_flat (the same values).
template <bool FLAT = false>
__device__ __forceinline__ void gate_head(const GateIn& p, int h, float& neg_a, float& dtb) {
  neg_a = -expf(FLAT ? ldp_flat(p.A_log, h, p.pdt, p.H) : ldp(p.A_log, h, p.pdt));
  dtb = FLAT ? ldp_flat(p.dt_bias, h, p.pdt, p.H) : ldp(p.dt_bias, h, p.pdt);
}
// g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) from the loaded
// values (neg_a = -exp(A_log))
__device__ __forceinline__ void gate_math(const GateIn& p, float neg_a, float dtb, float av,
                                          float bv, float& g, float& beta) {
  const float x = av + dtb;
  const float bx = p.spb * x;
  // both sides formed, then selected (no branch; the clamp changes nothing
  // where the log side is taken)
  const float lp = log1pf(expf(fminf(bx, p.spt))) / p.spb;
  const float sp = bx > p.spt ? x : lp;
  g = neg_a * sp;
  beta = 1.f / (1.f + expf(-bv));
}
template <bool FLAT = false>
__device__ __forceinline__ void gate_elem(const GateIn& p, long long i, float neg_a, float dtb,
                                          float& g, float& beta) {
  const float av = FLAT ? ldp_flat(p.a, i, p.adt, p.n) : ldp(p.a, i, p.adt);
  const float bv = FLAT ? ldp_flat(p.b, i, p.bdt, p.n) : (p.b ? ldp(p.b, i, p.bdt) : 0.f);
  gate_math(p, neg_a, dtb, av, bv, g, beta);
}
// gate_at's loads issued ahead of its math (gate_eval, the same values)
struct GateRaw {
  FlatRaw A, d, a, b;
};
__device__ __forceinline__ GateRaw gate_load(const GateIn& p, long long i, int h) {
  GateRaw r;
  r.A = ldp_flat_raw(p.A_log, h, p.pdt, p.H);
  r.d = ldp_flat_raw(p.dt_bias, h, p.pdt, p.H);
  r.a = ldp_flat_raw(p.a, i, p.adt, p.n);
  r.b = ldp_flat_raw(p.b, i, p.bdt, p.n);
  return r;
}
__device__ __forceinline__ void gate_eval(const GateIn& p, const GateRaw& r, float& g,
                                          float& beta) {
  const float neg_a = -expf(flat_value(r.A, p.pdt));
  gate_math(p, neg_a, flat_value(r.d, p.pdt), flat_value(r.a, p.adt), flat_value(r.b, p.bdt), g,
            beta);
}
__device__ __forceinline__ void gate_at(const GateIn& p, long long i, int h, float& g,
                                        float& beta) {
  float neg_a, dtb;
  gate_head(p, h, neg_a, dtb);
  gate_elem(p, i, neg_a, dtb, g, beta);
}


}  // namespace gdn

// ---- host side: error channel shared by every entry point -------------
namespace gdn_host {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
void launch_begin();
int check_launch(const char* what);
// [a, a + na) and [b, b + nb) share a byte (callers skip NULL pointers).
bool overlaps(const void* a, size_t na, const void* b, size_t nb);
}  // namespace gdn_host
