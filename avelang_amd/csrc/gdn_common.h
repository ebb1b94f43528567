// Shared device helpers for the gfx950 GDN kernels: bf16 packing, the
// 16x16x32 bf16 MFMA wrapper, and the thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/gdn.h"

namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;  // tokens per chunk of the prefill path
// Word 3 of a raw (stride 0) buffer resource on gfx950: out-of-range loads
// return 0 and out-of-range stores are dropped.
constexpr int kBufferFlags = 0x00020000;
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

// D = A B + C for fp32 16x16x4 (one block): lane l holds A[l % 16][l / 16]
// and B[l / 16][l % 16]; D has the same layout as the 16x16x32 bf16 form.
__device__ __forceinline__ f32x4 mfma4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

}  // namespace gdn

// ---- host side: error channel shared by every entry point -------------
namespace gdn_host {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
// [a, a + na) and [b, b + nb) share a byte (callers skip NULL pointers).
bool overlaps(const void* a, size_t na, const void* b, size_t nb);
}  // namespace gdn_host
