"""avelang_amd — MI355X-native (gfx950) gated-delta-net hot path.

Operators (FLA / Qwen3-Next argument lists):
    chunk_gated_delta_rule            chunked prefill (chunk 64, MFMA), differentiable
    chunk_gated_delta_rule_bwd        its gradients (q, k, v, g, beta, initial state)
    fused_recurrent_gated_delta_rule  token recurrence / decode (HBM-bound),
                                      optionally over a pool of state slots

Neighbours of the core in the Qwen3-Next layer (``layer_ops``):
    fused_gdn_gating (differentiable; fused_gdn_gating_bwd), l2norm_fwd,
    causal_conv1d_fn, causal_conv1d_update, rms_norm_gated

All call hand-written HIP kernels through the C ABI in include/gdn.h and
include/gdn_layer.h (``libgdn.so``, built by ``python -m avelang_amd.build``).
"""
from .gated_delta_rule import (  # noqa: F401
    chunk_bwd_workspace_bytes,
    chunk_gated_delta_rule,
    chunk_gated_delta_rule_bwd,
    chunk_gated_delta_rule_fwd_save,
    chunk_gated_delta_rule_gated,
    chunk_workspace_bytes,
    fused_recurrent_gated_delta_rule,
    fused_recurrent_gated_delta_rule_gated,
)
from .layer_ops import (  # noqa: F401
    causal_conv1d_fn,
    causal_conv1d_update,
    fused_gdn_gating,
    fused_gdn_gating_bwd,
    l2norm_fwd,
    rms_norm_gated,
)

__all__ = [
    "chunk_gated_delta_rule",
    "chunk_gated_delta_rule_bwd",
    "chunk_gated_delta_rule_fwd_save",
    "fused_recurrent_gated_delta_rule",
    "chunk_gated_delta_rule_gated",
    "fused_recurrent_gated_delta_rule_gated",
    "chunk_workspace_bytes",
    "chunk_bwd_workspace_bytes",
    "fused_gdn_gating",
    "fused_gdn_gating_bwd",
    "l2norm_fwd",
    "causal_conv1d_fn",
    "causal_conv1d_update",
    "rms_norm_gated",
]
