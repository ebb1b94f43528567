"""avelang_amd — MI355X-native (gfx950) gated-delta-net hot path.

Operators (FLA / Qwen3-Next argument lists):
    chunk_gated_delta_rule            chunked prefill (chunk 64, MFMA)
    fused_recurrent_gated_delta_rule  token recurrence / decode (HBM-bound)

Both call hand-written HIP kernels through the C ABI in include/gdn.h
(``libgdn.so``, built by ``python -m avelang_amd.build``).
"""
from .gated_delta_rule import (  # noqa: F401
    chunk_gated_delta_rule,
    chunk_workspace_bytes,
    fused_recurrent_gated_delta_rule,
)

__all__ = [
    "chunk_gated_delta_rule",
    "fused_recurrent_gated_delta_rule",
    "chunk_workspace_bytes",
]
