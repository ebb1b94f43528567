/*
 * gdn_layer.h — C ABI of the producer / consumer operators around the
 * gated-delta-net core in a Qwen3-Next linear-attention layer, for MI355X
 * (gfx950).  Same conventions as gdn.h: caller-owned device pointers,
 * nothing allocated or synchronised, work enqueued on `stream`, 0 / < 0
 * (argument error, nothing enqueued) / > 0 (hipError_t), gdn_last_error().
 *
 * The reference repository (848267592/avelang) has no counterpart for any
 * of these; their semantics follow the Qwen3-Next layer text of
 * transformers 5.15.0 models/qwen3_next/modeling_qwen3_next.py (cited as
 * TF:line), read as text only, and their argument lists follow the kernel
 * libraries that layer binds to (causal-conv1d's causal_conv1d_fn /
 * causal_conv1d_update, FLA's l2norm / fused gating / gated RMSNorm).
 *
 * Element types are passed as GDN_DTYPE_* codes.  Strides are in elements.
 */
#ifndef AVELANG_AMD_GDN_LAYER_H
#define AVELANG_AMD_GDN_LAYER_H

#include <stddef.h>
#include <stdint.h>

#include "gdn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_DTYPE_F32 0
#define GDN_DTYPE_BF16 1
#define GDN_DTYPE_F16 2

/*
 * Decay and write-strength gates from the layer's projections (TF:650-652):
 *   g    = -exp(A_log[h]) * softplus(a + dt_bias[h])
 *   beta = sigmoid(b)
 * softplus(x) = log(1 + exp(sp_beta x)) / sp_beta, or x where
 * sp_beta x > sp_threshold (torch.nn.functional.softplus).
 *   a, b      [rows, H] (a_dtype, b_dtype)      A_log, dt_bias [H] (p_dtype)
 *   g, beta   [rows, H] fp32 outputs (beta nullable: only g is written)
 */
int gdn_gating_fwd(const void* A_log, const void* a, const void* b, const void* dt_bias,
                   float* g, float* beta, long long rows, int H,
                   int a_dtype, int b_dtype, int p_dtype,
                   float sp_beta, float sp_threshold, void* stream);

/*
 * Backward of gdn_gating_fwd: what autograd through the layer's gating
 * expression (TF:650-652) gives, in one elementwise pass plus a per-head
 * sum.  From dg, dbeta [rows, H] fp32 (the core's gradients w.r.t. g, beta):
 *   da       [rows, H] (a_dtype) = dg * -exp(A_log) * softplus'(a + dt_bias)
 *   db       [rows, H] (b_dtype) = dbeta * beta * (1 - beta)
 *   ddt_bias [H] (p_dtype)       = sum over rows of da (fp32, before rounding)
 *   dA_log   [H] (p_dtype)       = sum over rows of dg * g
 * softplus'(x) = sigmoid(sp_beta x), or 1 where sp_beta x > sp_threshold
 * (torch's softplus backward).  db / dbeta are nullable together; dA_log
 * and ddt_bias are nullable.  The sums are deterministic (a fixed order, no
 * atomics).  workspace: gdn_gating_bwd_workspace_bytes(rows, H) bytes of
 * device memory (0 bytes: may be NULL).  0 < H <= 256.  No counterpart in
 * the reference (it has no GDN code); the layer's autograd is what it
 * replaces.
 */
size_t gdn_gating_bwd_workspace_bytes(long long rows, int H);
int gdn_gating_bwd(const void* A_log, const void* a, const void* b, const void* dt_bias,
                   const float* dg, const float* dbeta,
                   void* dA_log, void* da, void* db, void* ddt_bias,
                   long long rows, int H, int a_dtype, int b_dtype, int p_dtype,
                   float sp_beta, float sp_threshold,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Row L2 normalisation, y = x * rsqrt(sum(x^2) + eps) over D (TF:368-371).
 *   x, y [rows, D] contiguous, same dtype (f32 / bf16 / f16); D in {64, 128, 256}.
 * y may equal x.
 */
int gdn_l2norm_fwd(const void* x, void* y, long long rows, int D, float eps, int dtype,
                   void* stream);

/*
 * Causal depthwise convolution over time (TF:346-365; causal-conv1d's
 * causal_conv1d_fn):
 *   out[b, d, t] = act(bias[d] + sum_{j<W} w[d, j] * x[b, d, t - (W-1) + j])
 * with zeros (or initial_states) before the start of each sequence;
 * act = SiLU when silu != 0.
 *   x, out  [B, D, T] with element strides (x_sb, x_sd, x_st), (o_sb, o_sd, o_st);
 *           either channel-last (x_sd == o_sd == 1) or time-contiguous
 *           (x_st == o_st == 1); dtype f32 / bf16 / f16.
 *   weight  [D, W] contiguous, bias [D] nullable (w_dtype); W in {2, 3, 4}.
 *   seq_idx [B, T] int32 nullable (channel-last only): a token's window
 *           only reads tokens with the same seq_idx (packed varlen).
 *   initial_states [B, D, W-1] nullable, final_states [B, D, W-1]
 *           nullable (contiguous, x's dtype; channel-last only): the W-1
 *           inputs before / at the end of each batch row.
 */
int gdn_causal_conv1d_fwd(const void* x, const void* weight, const void* bias,
                          const int32_t* seq_idx, const void* initial_states,
                          void* final_states, void* out, int B, int D, int T, int W,
                          long long x_sb, long long x_sd, long long x_st,
                          long long o_sb, long long o_sd, long long o_st,
                          int silu, int dtype, int w_dtype, void* stream);

/*
 * One decode step of the causal convolution with its rolling input state
 * updated in place (TF:326-343; causal-conv1d's causal_conv1d_update):
 *   window = concat(conv_state[slot, d, :], x[b, d, 0:L])
 *   out[b, d, t] = act(bias[d] + sum_{j<W} w[d, j] * window[S + t - (W-1) + j])
 *   conv_state[slot, d, :] = window[L : L + S]
 *   x, out     [B, D, L] with element strides; L in [1, 64]
 *   conv_state [num_slots, D, S] contiguous, x's dtype; S in [W-1, 8]
 *   conv_state_indices [B] int32 nullable (slot = b when NULL); a slot
 *           outside [0, num_slots) marks a padding row: nothing is read or
 *           written for it.
 */
int gdn_causal_conv1d_update(const void* x, void* conv_state, const void* weight,
                             const void* bias, const int32_t* conv_state_indices, void* out,
                             int B, int D, int L, int W, int S, int num_slots,
                             long long x_sb, long long x_sd, long long x_st,
                             long long o_sb, long long o_sd, long long o_st,
                             int silu, int dtype, int w_dtype, void* stream);

/*
 * Gated RMSNorm applied to the core output (TF:58-74, call TF:693), norm
 * before gate, with the layer's rounding steps for low-precision inputs:
 *   n   = dtype(x * rsqrt(mean(x^2) + eps))
 *   out = dtype((weight * n) * silu(z))    (weight * n rounded to dtype
 *                                            when w_dtype == dtype)
 *   x, z, out [rows, D] contiguous (dtype), weight [D] (w_dtype);
 *   D in {64, 128, 256}.
 */
int gdn_rmsnorm_gated_fwd(const void* x, const void* z, const void* weight, void* out,
                          long long rows, int D, float eps, int dtype, int w_dtype,
                          void* stream);

/*
 * Fused recurrent gated delta rule over a pool of state slots (continuous
 * batching): as gdn_recurrent_fwd, but sequence n reads and writes state
 * slot state_indices[n] of h0 / ht, which are [num_slots, Hv, K, V].  A
 * slot outside [0, num_slots) marks a padding sequence: its state is not
 * touched and its output rows are not written.  ht may equal h0 (in place).
 * Sequences must not share a slot; the kernel checks this on the device:
 * every sequence whose slot another sequence also names leaves that slot
 * untouched and gets NaN output rows (so the pool is never written by two
 * workgroups at once, and the caller's mistake shows in o).
 */
int gdn_recurrent_fwd_indexed(const void* q, const void* k, const void* v,
                              const float* g, const float* beta,
                              const float* h0, float* ht, void* o,
                              const int32_t* cu_seqlens, const int32_t* state_indices,
                              int B, int T, int Hqk, int Hv, int K, int V, int N,
                              int num_slots, float scale, int use_qk_l2norm, void* stream);

/*
 * Speculative-decoding step over a state pool (draft tokens verified in one
 * call; the convention of the serving call site of fused_recurrent_gated_
 * delta_rule with a 2-D ssm_state_indices and num_accepted_tokens).
 *   state_indices        [N, index_stride] int32: the state after token t
 *                        (0-based within sequence n, t < index_stride) is
 *                        written to slot state_indices[n][t]; an entry outside
 *                        [0, num_slots) skips that write.
 *   num_accepted_tokens  [N] int32, nullable: sequence n starts from slot
 *                        state_indices[n][num_accepted_tokens[n] - 1] (the
 *                        state after the last draft token the previous step
 *                        accepted); NULL starts from state_indices[n][0].  An
 *                        initial slot outside the pool (or an accepted count
 *                        outside [1, index_stride]) marks a padding sequence:
 *                        nothing of it is read or written.
 *   pool                 [num_slots, Hv, K, V] fp32, read and written in place.
 * Without cu_seqlens every sequence has T tokens and T <= index_stride is
 * required; with cu_seqlens, tokens past index_stride advance the state
 * without writing it.  Sequences must not share slots (a row may repeat its
 * own): checked on the device as for gdn_recurrent_fwd_indexed, over the
 * entries each sequence reads or writes (its initial entry and those of its
 * tokens) -- every sequence involved writes no state and gets NaN outputs.
 */
int gdn_recurrent_fwd_spec(const void* q, const void* k, const void* v,
                           const float* g, const float* beta, float* pool, void* o,
                           const int32_t* cu_seqlens, const int32_t* state_indices,
                           int index_stride, const int32_t* num_accepted_tokens,
                           int B, int T, int Hqk, int Hv, int K, int V, int N,
                           int num_slots, float scale, int use_qk_l2norm, void* stream);

/*
 * The gating fused into the core (TF:650-652 feeding :658-683): g and beta
 * are formed from (A_log, a, b, dt_bias) inside the kernels exactly as
 * gdn_gating_fwd forms them (one shared definition, the same bits), so no
 * fp32 g / beta tensor is written and read back, and the gating launch
 * goes away.  Arguments as gdn_gating_fwd's (a, b [B, T, Hv]) followed by
 * the core's.  No counterpart in the reference (it has no GDN code); the
 * layer's own call sequence gating -> core is what they replace.
 *
 * gdn_chunk_fwd_gating: gdn_chunk_fwd with g, beta replaced; workspace of
 *   gdn_chunk_workspace_bytes.
 * gdn_recurrent_fwd_gating: state_indices NULL: gdn_recurrent_fwd (h0 ->
 *   ht, num_slots ignored); state_indices set: gdn_recurrent_fwd_indexed
 *   (h0 / ht are the [num_slots, Hv, K, V] pool).
 */
int gdn_chunk_fwd_gating(const void* q, const void* k, const void* v,
                         const void* A_log, const void* a, const void* b, const void* dt_bias,
                         int a_dtype, int b_dtype, int p_dtype, float sp_beta,
                         float sp_threshold,
                         const float* h0, float* ht, void* o, const int32_t* cu_seqlens,
                         int B, int T, int Hqk, int Hv, int K, int V, int N,
                         float scale, int use_qk_l2norm,
                         void* workspace, size_t workspace_bytes, void* stream);
int gdn_recurrent_fwd_gating(const void* q, const void* k, const void* v,
                             const void* A_log, const void* a, const void* b,
                             const void* dt_bias, int a_dtype, int b_dtype, int p_dtype,
                             float sp_beta, float sp_threshold,
                             const float* h0, float* ht, void* o, const int32_t* cu_seqlens,
                             const int32_t* state_indices,
                             int B, int T, int Hqk, int Hv, int K, int V, int N, int num_slots,
                             float scale, int use_qk_l2norm, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AVELANG_AMD_GDN_LAYER_H */
