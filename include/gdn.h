/*
 * gdn.h — C ABI of the MI355X (gfx950) gated-delta-net hot path.
 *
 * The reference repository (848267592/avelang) ships no gated-delta-rule
 * code; its only kernel-library entry point is the Python wrapper
 * `gemm_pipeline_transposed_b` (python/avelang_kernels/amdgpu_gemm.py:458-494)
 * launched through a generated C launcher that takes raw device pointers,
 * scalars and torch's current stream (python/avelang/backends/amdgpu/
 * driver.py:220-392, stream getter backends/driver.py:24-30).  These entry
 * points take the place of that launcher for the two GDN operators that
 * Qwen3-Next calls (transformers modeling_qwen3_next.py:658-683):
 *   chunk_gated_delta_rule            -> gdn_chunk_fwd (backward: gdn_chunk_bwd)
 *   fused_recurrent_gated_delta_rule  -> gdn_recurrent_fwd
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers; the caller owns every buffer.  Nothing
 *     here allocates device memory or synchronises; work is enqueued on
 *     `stream` (a hipStream_t; NULL = the legacy default stream).
 *   - Layouts (row-major, contiguous):
 *       q, k   [B, T, Hqk, K]  bf16
 *       v, o   [B, T, Hv,  V]  bf16
 *       g, beta[B, T, Hv]      fp32   (g = natural-log decay, applied as exp(g))
 *       state  [N, Hv, K, V]   fp32   (S stored K-major: o_t = scale * S^T q_t)
 *     v-head h reads qk-head h / (Hv / Hqk).
 *   - cu_seqlens (nullable) is an int32 device array [N+1] of packed
 *     sequence offsets; it requires B == 1.  Without it N == B and every
 *     batch row is one sequence of length T.  Contract: cu_seqlens[0] == 0,
 *     non-decreasing, cu_seqlens[N] == T.  Being device memory it is not
 *     read on the host; gdn_cu_seqlens_check() makes the same check on a
 *     host copy.  The chunked entry points (gdn_chunk_fwd, _fwd_save,
 *     _bwd) also check it on the device: on a violation every sequence is
 *     treated as empty -- o and the gradients are zero-filled, ht = h0 and
 *     dh0 = dht -- and the call still returns 0.  The recurrent entry points
 *     clamp each sequence's range to [0, T] instead.
 *   - Return value: 0 = success; < 0 = argument error (nothing enqueued);
 *     > 0 = a hipError_t from a launch.  gdn_last_error() gives a
 *     thread-local message for the last failing call of this thread.
 *   - Supported head sizes: K in {64, 128}; V in {64, 128}.
 */
#ifndef AVELANG_AMD_GDN_H
#define AVELANG_AMD_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Argument-error codes (negative). */
#define GDN_OK 0
#define GDN_ERR_NULL (-1)        /* required pointer is NULL            */
#define GDN_ERR_SHAPE (-2)       /* unsupported or inconsistent shape   */
#define GDN_ERR_SEQLENS (-3)     /* cu_seqlens / N inconsistent         */
#define GDN_ERR_WORKSPACE (-4)   /* workspace NULL or too small         */
#define GDN_ERR_ALIAS (-5)       /* forbidden buffer aliasing           */

/*
 * Chunked prefill (chunk = 64 tokens).  Replaces the launcher call an
 * avelang_kernels `chunk_gated_delta_rule` op would make (convention:
 * amdgpu_gemm.py:488-493 -> driver.py:324-343); operator semantics as
 * modeling_qwen3_next.py:374-453.
 *
 *   h0  nullable: initial state [N, Hv, K, V]; NULL = zeros.
 *   ht  nullable: final state   [N, Hv, K, V]; NULL = not written.
 *       ht may equal h0 (in-place update); any other overlap is an error.
 *   use_qk_l2norm != 0: q and k are L2-normalised over K (eps 1e-6) and
 *       rounded to bf16 before use.
 *   workspace: device scratch of at least gdn_chunk_workspace_bytes(...).
 * Precision: the sequential state products take fp16 operands (one MFMA
 * pass, fp32 accumulation and fp32 state), so q, k, the state and v-sized
 * intermediates must stay inside fp16's range (|x| < 65504); l2-normalised
 * q / k (or use_qk_l2norm) and the v of a Qwen3-Next layer are orders of
 * magnitude inside it.  The final state is within ~4e-4 relative Frobenius
 * of the exact recurrence at any length.  Without use_qk_l2norm the output's
 * q.S term is a bf16 MFMA product (q as given, the state rounded to bf16);
 * with it an fp16 one (the normalised q as fp16); gdn_chunk_fwd_save gives
 * the same o as gdn_chunk_fwd either way.
 */
int gdn_chunk_fwd(const void* q, const void* k, const void* v,
                  const float* g, const float* beta,
                  const float* h0, float* ht, void* o,
                  const int32_t* cu_seqlens,
                  int B, int T, int Hqk, int Hv, int K, int V, int N,
                  float scale, int use_qk_l2norm,
                  void* workspace, size_t workspace_bytes,
                  void* stream);

/* Bytes of device workspace gdn_chunk_fwd needs for these sizes
 * (an upper bound when cu_seqlens is used: T/64 + N chunks). */
size_t gdn_chunk_workspace_bytes(int B, int T, int Hqk, int Hv, int K, int V,
                                 int N, int has_cu_seqlens, int use_qk_l2norm);

/* Bytes of device scratch gdn_chunk_fwd_noalloc owns on every GPU. */
#define GDN_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/*
 * gdn_chunk_fwd without a workspace argument: the library's own device
 * scratch (a fixed array of GDN_NOALLOC_SCRATCH_BYTES = 32 MiB per GPU)
 * takes its place, so the call allocates nothing -- no hipMalloc, no
 * hipFree, no allocating library routine.  No counterpart in the
 * reference; it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).
 * The array is part of libgdn.so's device code object: every process that
 * loads the library holds those 32 MiB on every GPU it uses, until it ends,
 * whether or not it calls this entry point.
 * Problems whose gdn_chunk_workspace_bytes(...) exceeds 32 MiB (about 5,300
 * tokens at 32 v-heads / 16 qk-heads, K = V = 128; about 2,300 with
 * use_qk_l2norm, whose chain reads fp16 copies of the normalised q, k rows
 * from the workspace) are rejected with
 * GDN_ERR_WORKSPACE before anything is enqueued.  Every call on one GPU
 * shares that GPU's scratch: calls that overlap on one GPU (different
 * streams, or host threads) race and must be serialised by the caller.
 * The scratch's device address is looked up on a device's first call
 * (in relaxed stream-capture mode, so that first call may itself be under
 * capture).
 */
int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v,
                          const float* g, const float* beta,
                          const float* h0, float* ht, void* o,
                          const int32_t* cu_seqlens,
                          int B, int T, int Hqk, int Hv, int K, int V, int N,
                          float scale, int use_qk_l2norm,
                          void* stream);

/*
 * Training forward: gdn_chunk_fwd's results (o, ht) plus, in `workspace`
 * (at least gdn_chunk_bwd_workspace_bytes(...)), everything gdn_chunk_bwd
 * needs, so that a later gdn_chunk_bwd(..., saved = 1, same workspace) on
 * the same inputs skips its forward recomputation.  The forward half of an
 * autograd chunk_gated_delta_rule (FLA's autograd function; Qwen3-Next trains
 * through it, modeling_qwen3_next.py:672-683); no reference counterpart.
 */
int gdn_chunk_fwd_save(const void* q, const void* k, const void* v,
                       const float* g, const float* beta,
                       const float* h0, float* ht, void* o,
                       const int32_t* cu_seqlens,
                       int B, int T, int Hqk, int Hv, int K, int V, int N,
                       float scale, int use_qk_l2norm,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * Fused recurrent form (decode: T == 1 per sequence; also multi-token).
 * Replaces the launcher call of `fused_recurrent_gated_delta_rule`
 * (semantics modeling_qwen3_next.py:456-503).  The state tile of each
 * (sequence, v-head) is streamed once from HBM, advanced through that
 * sequence's tokens in registers, and written once.
 *
 *   h0 nullable (zeros); ht nullable (not written); ht == h0 updates the
 *   state in place (the decode configuration).
 */
int gdn_recurrent_fwd(const void* q, const void* k, const void* v,
                      const float* g, const float* beta,
                      const float* h0, float* ht, void* o,
                      const int32_t* cu_seqlens,
                      int B, int T, int Hqk, int Hv, int K, int V, int N,
                      float scale, int use_qk_l2norm,
                      void* stream);

/*
 * Chunked backward (chunk = 64 tokens): gradients of gdn_chunk_fwd's o and
 * final state with respect to q, k, v, g, beta and h0.  Replaces the
 * backward launch of FLA's autograd chunk_gated_delta_rule (the operator
 * Qwen3-Next trains through, modeling_qwen3_next.py:672-683); the
 * reference repository has no counterpart (its kernel library,
 * python/avelang_kernels/, is forward-only and holds one GEMM).
 *
 * Recomputes the forward from (q, k, v, g, beta, h0) -- or takes it from a
 * gdn_chunk_fwd_save workspace (saved != 0) -- then runs the state gradient
 * backwards over the chunks and forms every chunk's local gradients in
 * parallel.
 *
 *   dO    [B, T, Hv, V] bf16: dL/do.
 *   dht   nullable: dL/d(final state) [N, Hv, K, V] fp32; NULL = zeros.
 *   dq, dk [B, T, Hqk, K] bf16 (summed over each qk-head's v-heads);
 *   dv    [B, T, Hv, V] bf16;  dg, dbeta [B, T, Hv] fp32.
 *   dh0   nullable: dL/dh0 [N, Hv, K, V] fp32 (written even when h0 is NULL:
 *         the gradient with respect to a zero initial state).
 *   use_qk_l2norm != 0: the forward normalised q and k; dq and dk are the
 *         gradients with respect to the raw (unnormalised) q and k.
 *   saved != 0: `workspace` holds what gdn_chunk_fwd_save left there for
 *         these same inputs; the forward recomputation is skipped.  0: the
 *         forward is recomputed from (q, k, v, g, beta, h0).
 *   workspace: at least gdn_chunk_bwd_workspace_bytes(...).
 * Every output is fully overwritten (no accumulation into it).
 */
int gdn_chunk_bwd(const void* q, const void* k, const void* v,
                  const float* g, const float* beta, const float* h0,
                  const void* dO, const float* dht,
                  void* dq, void* dk, void* dv, float* dg, float* dbeta, float* dh0,
                  const int32_t* cu_seqlens,
                  int B, int T, int Hqk, int Hv, int K, int V, int N,
                  float scale, int use_qk_l2norm, int saved,
                  void* workspace, size_t workspace_bytes,
                  void* stream);

/* Bytes of device workspace gdn_chunk_bwd (and gdn_chunk_fwd_save) need. */
size_t gdn_chunk_bwd_workspace_bytes(int B, int T, int Hqk, int Hv, int K, int V,
                                     int N, int has_cu_seqlens, int use_qk_l2norm);

/*
 * Host-side check of the cu_seqlens contract above on a host array [N+1]:
 * GDN_OK, or GDN_ERR_SEQLENS naming the first violation (gdn_last_error()).
 * The same conditions the chunked kernels check on the device.  No
 * counterpart in the reference (it has no varlen plumbing); callers that
 * hold cu_seqlens on the host use it to get an error instead of the
 * device-side empty-sequence fallback.
 */
int gdn_cu_seqlens_check(const int32_t* cu_seqlens, int N, int total_tokens);

/* Thread-local message describing the last failure (never NULL). */
const char* gdn_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int gdn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* AVELANG_AMD_GDN_H */
