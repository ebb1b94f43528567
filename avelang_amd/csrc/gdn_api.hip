// Host-side argument validation and the thread-local error channel of the
// C ABI.  Error behaviour mirrors the reference's kernel-library wrapper
// (python/avelang_kernels/amdgpu_gemm.py:463-486: shape/dtype problems are
// argument errors raised before any launch) and its launcher (python/avelang/
// backends/amdgpu/driver.py:125-138: HIP failures surface as errors carrying
// the HIP message).  Here the former are negative return codes, the latter
// positive hipError_t values; the message is kept per thread.
#include <cstdio>
#include <string>

#include "gdn_chunk.h"
#include "gdn_common.h"

namespace gdn_host {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// A launch error already pending on this thread when an entry point starts
// belongs to earlier work (another library's launch, say): it is taken off
// the thread before this library's launches, so that check_launch reports
// only the entry point's own.
void launch_begin() { (void)hipGetLastError(); }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    g_last_error = std::string(what) + ": HIP error " + std::to_string((int)err) + " (" +
                   hipGetErrorString(err) + ")";
    return (int)err;
  }
  return GDN_OK;
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + nb && pb < pa + na;
}

int validate_common(const void* q, const void* k, const void* v, const float* g,
                    const float* beta, const float* h0, const float* ht, const void* o,
                    const int32_t* cu, int B, int T, int Hqk, int Hv, int K, int V, int N) {
  if (B < 0 || T < 0 || Hqk <= 0 || Hv <= 0 || N < 0)
    return fail(GDN_ERR_SHAPE, "sizes must be non-negative (Hqk, Hv > 0)");
  if (Hv % Hqk != 0)
    return fail(GDN_ERR_SHAPE, "Hv (" + std::to_string(Hv) + ") must be a multiple of Hqk (" +
                                   std::to_string(Hqk) + ")");
  if (!((K == 64 || K == 128) && (V == 64 || V == 128)))
    return fail(GDN_ERR_SHAPE, "unsupported head sizes K=" + std::to_string(K) +
                                   " V=" + std::to_string(V) + " (K, V in {64, 128})");
  const long long tokens = (long long)B * T;
  if (tokens * Hv * (long long)V >= (1LL << 40))
    return fail(GDN_ERR_SHAPE, "problem too large");
  if (cu) {
    if (B != 1) return fail(GDN_ERR_SEQLENS, "cu_seqlens requires B == 1");
    if (N < 1 && T > 0) return fail(GDN_ERR_SEQLENS, "cu_seqlens requires N >= 1");
  } else if (N != B) {
    return fail(GDN_ERR_SEQLENS, "without cu_seqlens N must equal B");
  }
  if (tokens > 0 && (!q || !k || !v || !g || !beta || !o))
    return fail(GDN_ERR_NULL, "q, k, v, g, beta and o must be non-NULL");
  if (ht && h0 && ht != h0) {
    const size_t sb = (size_t)N * Hv * K * V * sizeof(float);
    if (overlaps(h0, sb, ht, sb))
      return fail(GDN_ERR_ALIAS, "ht must equal h0 exactly or not overlap it");
  }
  if (o && tokens > 0) {
    const size_t ob = (size_t)tokens * Hv * V * 2;
    const size_t qb = (size_t)tokens * Hqk * K * 2;
    if (overlaps(o, ob, q, qb) || overlaps(o, ob, k, qb) || overlaps(o, ob, v, ob))
      return fail(GDN_ERR_ALIAS, "o must not overlap q, k or v");
  }
  return GDN_OK;
}

// Arguments of the gating the fused entry points compute inside (a and b
// are null-checked by validate_common in place of g and beta).
int validate_gate(const char* name, const void* A_log, const void* dt_bias, int a_dtype,
                  int b_dtype, int p_dtype, float sp_beta, long long tokens) {
  if (!gdn::dtype_ok(a_dtype) || !gdn::dtype_ok(b_dtype) || !gdn::dtype_ok(p_dtype))
    return fail(GDN_ERR_SHAPE, std::string(name) + ": unsupported dtype code");
  if (!(sp_beta > 0.f)) return fail(GDN_ERR_SHAPE, std::string(name) + ": softplus beta must be > 0");
  if (tokens > 0 && (!A_log || !dt_bias))
    return fail(GDN_ERR_NULL, std::string(name) + ": A_log and dt_bias must be non-NULL");
  return GDN_OK;
}

// The fused kernels address a, b with 32-bit byte offsets (4 bytes per element).
int validate_gate_size(const char* name, long long elements) {
  if (elements * 4 >= (1LL << 31))
    return fail(GDN_ERR_SHAPE, std::string(name) + ": a, b too large for the fused gating");
  return GDN_OK;
}

}  // namespace gdn_host

extern "C" const char* gdn_last_error(void) { return gdn_host::g_last_error.c_str(); }

extern "C" int gdn_abi_version(void) { return 101; }

// Host-side form of the device check the chunked kernels make (declared in
// gdn.h): the contract on cu_seqlens.
extern "C" int gdn_cu_seqlens_check(const int32_t* cu_seqlens, int N, int total_tokens) {
  if (!cu_seqlens) return gdn_host::fail(GDN_ERR_NULL, "gdn_cu_seqlens_check: cu_seqlens is NULL");
  if (N < 0 || total_tokens < 0)
    return gdn_host::fail(GDN_ERR_SHAPE, "gdn_cu_seqlens_check: N and total_tokens must be >= 0");
  static const char* what[] = {"", "cu_seqlens[0] must be 0", "cu_seqlens must be non-decreasing",
                               "cu_seqlens[N] must equal the packed token count"};
  const int v = gdn::cu_seqlens_violation(cu_seqlens, N, total_tokens);
  return v ? gdn_host::fail(GDN_ERR_SEQLENS, std::string("gdn_cu_seqlens_check: ") + what[v]) : GDN_OK;
}
