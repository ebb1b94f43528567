"""Gated delta rule operators for MI355X (gfx950).

Python operator surface of the Qwen3-Next gated-delta-net hot path, in the
shape of the reference's kernel-library wrappers
(python/avelang_kernels/amdgpu_gemm.py:458-494): validate dtypes and shapes
and raise ``ValueError`` before anything is launched, allocate outputs on
the inputs' device, and launch asynchronously on torch's current stream
(python/avelang/backends/driver.py:24-30).  The kernels are the hand-written
HIP code of ``avelang_amd/csrc`` behind the C ABI of ``include/gdn.h``; there
is no fallback path.

Layouts (FLA / transformers convention, modeling_qwen3_next.py:391-393):
    q, k  [B, T, Hqk, K]  bf16        v, o  [B, T, Hv, V]  bf16
    g, beta [B, T, Hv]    fp32        state [N, Hv, K, V]  fp32
v-head h reads qk-head h // (Hv // Hqk).  The state is stored K-major, so
o_t = scale * S_t^T q_t; the recurrence written V-major,
S <- e^g S (I - beta k k^T) + beta v k^T, o = S q, is the same operator.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch.autograd.function import once_differentiable

from . import _native
from .layer_ops import fused_gdn_gating

__all__ = [
    "chunk_gated_delta_rule",
    "chunk_gated_delta_rule_bwd",
    "chunk_gated_delta_rule_fwd_save",
    "fused_recurrent_gated_delta_rule",
    "chunk_workspace_bytes",
    "chunk_gated_delta_rule_gated",
    "fused_recurrent_gated_delta_rule_gated",
    "chunk_bwd_workspace_bytes",
]

CHUNK_SIZE = 64
_HEAD_SIZES = (64, 128)


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _check_inputs(q, k, v, g, beta, initial_state, cu_seqlens, name, convert_gates=True):
    for nm, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"{name}: {nm} must be a torch.Tensor")
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name}: {nm} must have dtype torch.bfloat16, got {t.dtype}.")
        if t.dim() != 4:
            raise ValueError(f"{name}: {nm} must be 4-D [B, T, H, D], got {tuple(t.shape)}.")
    B, T, Hqk, K = q.shape
    if tuple(k.shape) != (B, T, Hqk, K):
        raise ValueError(f"{name}: k must have shape {tuple(q.shape)}, got {tuple(k.shape)}.")
    if tuple(v.shape[:2]) != (B, T):
        raise ValueError(f"{name}: v must have shape [B, T, Hv, V] with B, T = {B}, {T}.")
    Hv, V = v.shape[2], v.shape[3]
    if Hqk == 0 or Hv % Hqk != 0:
        raise ValueError(f"{name}: v-heads ({Hv}) must be a multiple of qk-heads ({Hqk}).")
    if K not in _HEAD_SIZES or V not in _HEAD_SIZES:
        raise ValueError(f"{name}: head sizes K={K}, V={V} unsupported (each in {_HEAD_SIZES}).")
    for nm, t in (("g", g), ("beta", beta)):
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"{name}: {nm} must be a torch.Tensor")
        if tuple(t.shape) != (B, T, Hv):
            raise ValueError(f"{name}: {nm} must have shape {(B, T, Hv)}, got {tuple(t.shape)}.")
        if not t.is_floating_point():
            raise ValueError(f"{name}: {nm} must be floating point, got {t.dtype}.")
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError(f"{name}: cu_seqlens requires batch size 1, got {B}.")
        if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
            raise ValueError(f"{name}: cu_seqlens must be 1-D with at least 2 entries.")
        if cu_seqlens.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name}: cu_seqlens must be int32 or int64, got {cu_seqlens.dtype}.")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError(f"{name}: tensors must be on a ROCm (cuda) device, got {dev}.")
    for nm, t in (("k", k), ("v", v), ("g", g), ("beta", beta)):
        if t.device != dev:
            raise ValueError(f"{name}: {nm} must be on {dev}, got {t.device}.")

    if cu_seqlens is not None:
        N = cu_seqlens.numel() - 1
        if cu_seqlens.device.type == "cpu":
            # the library's own check of the contract (the chunked kernels
            # repeat it on the device, where a violation empties every
            # sequence instead of raising)
            c32 = cu_seqlens.to(torch.int32).contiguous()
            lib = _native.lib()
            if lib.gdn_cu_seqlens_check(c32.data_ptr(), N, T) != 0:
                raise ValueError(f"{name}: {lib.gdn_last_error().decode()} (T={T}).")
        elif cu_seqlens.device != dev:
            raise ValueError(f"{name}: cu_seqlens must be on {dev} or the CPU.")
        cu = cu_seqlens.to(device=dev, dtype=torch.int32, non_blocking=True).contiguous()
    else:
        N = B
        cu = None

    if initial_state is not None:
        if tuple(initial_state.shape) != (N, Hv, K, V):
            raise ValueError(f"{name}: initial_state must have shape {(N, Hv, K, V)}, "
                             f"got {tuple(initial_state.shape)}.")
        if initial_state.dtype != torch.float32:
            raise ValueError(f"{name}: initial_state must be torch.float32, got {initial_state.dtype}.")
        if initial_state.device != dev:
            raise ValueError(f"{name}: initial_state must be on {dev}.")
    if convert_gates:
        g = g.to(torch.float32).contiguous()
        beta = beta.to(torch.float32).contiguous()
    else:   # the gating inputs a, b of the fused entry points, in their own dtype
        g, beta = g.contiguous(), beta.contiguous()
    return (q.contiguous(), k.contiguous(), v.contiguous(), g, beta, cu,
            (B, T, Hqk, Hv, K, V, N))


def chunk_workspace_bytes(B: int, T: int, Hqk: int, Hv: int, K: int, V: int, N: int,
                          has_cu_seqlens: bool, use_qk_l2norm: bool = False) -> int:
    """Device scratch bytes ``chunk_gated_delta_rule`` needs (gdn_chunk_workspace_bytes)."""
    return int(_native.lib().gdn_chunk_workspace_bytes(
        B, T, Hqk, Hv, K, V, N, int(has_cu_seqlens), int(use_qk_l2norm)))


def chunk_bwd_workspace_bytes(B: int, T: int, Hqk: int, Hv: int, K: int, V: int, N: int,
                              has_cu_seqlens: bool, use_qk_l2norm: bool = False) -> int:
    """Device scratch bytes ``chunk_gated_delta_rule_bwd`` needs (gdn_chunk_bwd_workspace_bytes)."""
    return int(_native.lib().gdn_chunk_bwd_workspace_bytes(
        B, T, Hqk, Hv, K, V, N, int(has_cu_seqlens), int(use_qk_l2norm)))


def chunk_gated_delta_rule_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    do: torch.Tensor,
    dht: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    *,
    workspace: Optional[torch.Tensor] = None,
    saved: bool = False,
):
    """Gradients of ``chunk_gated_delta_rule`` (gdn_chunk_bwd).

    ``do`` is dL/do (bf16, the shape of v); ``dht`` (nullable) is dL/d(final
    state).  Returns ``(dq, dk, dv, dg, dbeta, dh0)``: dq, dk, dv in bf16,
    dg, dbeta in fp32, dh0 fp32 (``None`` without ``initial_state``).  The
    forward is recomputed from the inputs; nothing is kept from the forward
    call -- unless ``saved``: then ``workspace`` must be the one a training
    forward (``chunk_gated_delta_rule_fwd_save``) filled for these same
    inputs, and the recomputation is skipped.  With
    ``use_qk_l2norm_in_kernel`` dq and dk are gradients with respect to the
    raw q and k.
    """
    name = "chunk_gated_delta_rule_bwd"
    q, k, v, g, beta, cu, (B, T, Hqk, Hv, K, V, N) = _check_inputs(
        q, k, v, g, beta, initial_state, cu_seqlens, name)
    if scale is None:
        scale = K ** -0.5
    dev = q.device
    if (not isinstance(do, torch.Tensor) or do.shape != v.shape or do.dtype != torch.bfloat16
            or do.device != dev):
        raise ValueError(f"{name}: do must be a bf16 tensor of shape {tuple(v.shape)} on {dev}.")
    do = do.contiguous()
    if dht is not None:
        if (tuple(dht.shape) != (N, Hv, K, V) or dht.dtype != torch.float32
                or dht.device != dev):
            raise ValueError(f"{name}: dht must be fp32 {(N, Hv, K, V)} on {dev}.")
        dht = dht.contiguous()
    h0 = initial_state.contiguous() if initial_state is not None else None
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = torch.empty((B, T, Hv), dtype=torch.float32, device=dev)
    dbeta = torch.empty((B, T, Hv), dtype=torch.float32, device=dev)
    dh0 = torch.empty((N, Hv, K, V), dtype=torch.float32, device=dev) if h0 is not None else None
    nbytes = chunk_bwd_workspace_bytes(B, T, Hqk, Hv, K, V, N, cu is not None,
                                       use_qk_l2norm_in_kernel)
    if workspace is None:
        if saved:
            raise ValueError(f"{name}: saved=True needs the training forward's workspace.")
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < nbytes or workspace.device != dev:
        raise ValueError(f"{name}: workspace must be >= {nbytes} bytes on {dev}.")
    rc = _native.lib().gdn_chunk_bwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), _ptr(h0),
        do.data_ptr(), _ptr(dht),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), dbeta.data_ptr(), _ptr(dh0),
        _ptr(cu), B, T, Hqk, Hv, K, V, N, float(scale), int(bool(use_qk_l2norm_in_kernel)),
        int(bool(saved)), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        _stream_ptr(dev))
    _native.check(rc, name)
    return dq, dk, dv, dg, dbeta, dh0


def chunk_gated_delta_rule_fwd_save(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    *,
    workspace: Optional[torch.Tensor] = None,
):
    """Training forward (gdn_chunk_fwd_save): ``(o, final_state, workspace)``.

    ``o`` and ``final_state`` equal ``chunk_gated_delta_rule``'s; the
    returned workspace (``chunk_bwd_workspace_bytes`` bytes) holds what
    ``chunk_gated_delta_rule_bwd(..., workspace=ws, saved=True)`` needs for
    these same inputs.
    """
    if workspace is None:
        B, T, Hqk, K = q.shape
        Hv, V = v.shape[2], v.shape[3]
        N = B if cu_seqlens is None else cu_seqlens.numel() - 1
        nbytes = chunk_bwd_workspace_bytes(B, T, Hqk, Hv, K, V, N, cu_seqlens is not None,
                                           use_qk_l2norm_in_kernel)
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    o, ht = _chunk_fwd(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
                       use_qk_l2norm_in_kernel, save_workspace=workspace)
    return o, ht, workspace


# Default of chunk_gated_delta_rule's save_for_backward: the autograd forward
# keeps the backward's workspace (chunk_bwd_workspace_bytes: chunk-start
# states, deltas, the prep's fragments and fp16 K / Q copies -- about 160 KB
# per chunk and v-head, 622 MB for a T = 8192, 32-v-head layer) alive until
# the backward, which then skips the forward recomputation.  False: keep
# only the inputs and recompute (the backward then takes ~0.2 ms more at that
# shape).
SAVE_FORWARD_FOR_BACKWARD = True


class _ChunkGatedDeltaRule(torch.autograd.Function):
    """Autograd form of chunk_gated_delta_rule: forward gdn_chunk_fwd_save
    (or gdn_chunk_fwd), backward gdn_chunk_bwd (saved = 1, or recomputing)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
                use_qk_l2norm_in_kernel, save_for_backward):
        ws = None
        if save_for_backward:
            B, T, Hqk, K = q.shape
            Hv, V = v.shape[2], v.shape[3]
            N = B if cu_seqlens is None else cu_seqlens.numel() - 1
            nbytes = chunk_bwd_workspace_bytes(B, T, Hqk, Hv, K, V, N, cu_seqlens is not None,
                                               use_qk_l2norm_in_kernel)
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        o, ht = _chunk_fwd(q, k, v, g, beta, scale, initial_state, output_final_state,
                           cu_seqlens, use_qk_l2norm_in_kernel, save_workspace=ws)
        ctx.ws = ws
        ctx.save_for_backward(q, k, v, g, beta, initial_state, cu_seqlens)
        ctx.scale = scale
        ctx.l2 = use_qk_l2norm_in_kernel
        ctx.g_dtype, ctx.beta_dtype = g.dtype, beta.dtype
        ctx.has_ht = output_final_state
        if output_final_state:
            return o, ht
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, do, dht=None):
        q, k, v, g, beta, h0, cu = ctx.saved_tensors
        if dht is not None and not ctx.has_ht:
            dht = None
        ws, ctx.ws = ctx.ws, None
        dq, dk, dv, dg, db, dh0 = chunk_gated_delta_rule_bwd(
            q, k, v, g, beta, do.to(torch.bfloat16), dht.float() if dht is not None else None,
            ctx.scale, h0, cu, ctx.l2, workspace=ws, saved=ws is not None)
        return (dq, dk, dv, dg.to(ctx.g_dtype), db.to(ctx.beta_dtype), None, dh0, None, None,
                None, None)


def chunk_gated_delta_rule(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    *,
    workspace: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    final_state: Optional[torch.Tensor] = None,
    save_for_backward: Optional[bool] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Chunked (C = 64) gated-delta-rule prefill on gfx950.

    Semantics of torch_chunk_gated_delta_rule (modeling_qwen3_next.py:374-453)
    with FLA's argument list.  Returns ``(o, final_state)``; ``final_state``
    is ``None`` unless ``output_final_state``.  ``workspace`` (uint8, at least
    ``chunk_workspace_bytes(...)``), ``out`` and ``final_state`` may be passed
    to avoid allocation; ``final_state`` may be ``initial_state`` itself.
    With ``use_qk_l2norm_in_kernel`` q and k are L2-normalised (eps 1e-6)
    and rounded to bf16 before use, as FLA's separate l2norm pass does.
    The sequential state products run on fp16 operands (fp32 state and
    accumulation): q, k and v must stay inside fp16's range, which
    l2-normalised q / k and a layer's v do by orders of magnitude.

    Differentiable: when any of q, k, v, g, beta, initial_state requires
    grad (and grad mode is on) the call goes through an autograd function
    whose backward is ``chunk_gated_delta_rule_bwd`` (gdn_chunk_bwd).
    ``save_for_backward`` (default: the module's SAVE_FORWARD_FOR_BACKWARD)
    chooses, for that call, between keeping the backward's workspace from
    the forward (``chunk_bwd_workspace_bytes(...)`` bytes held until the
    backward, 622 MB at T = 8192 with 32 v-heads; the backward skips the
    recomputation) and keeping only the inputs (the backward recomputes).
    """
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q, k, v, g, beta, initial_state)):
        if out is not None or workspace is not None or final_state is not None:
            raise ValueError("chunk_gated_delta_rule: out / workspace / final_state buffers "
                             "are not supported when gradients are required.")
        if scale is None:
            scale = q.shape[-1] ** -0.5
        save = SAVE_FORWARD_FOR_BACKWARD if save_for_backward is None else bool(save_for_backward)
        res = _ChunkGatedDeltaRule.apply(q, k, v, g, beta, float(scale), initial_state,
                                         bool(output_final_state), cu_seqlens,
                                         bool(use_qk_l2norm_in_kernel), save)
        return (res[0], res[1]) if output_final_state else (res, None)
    return _chunk_fwd(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
                      use_qk_l2norm_in_kernel, workspace=workspace, out=out,
                      final_state=final_state)


def _chunk_fwd(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
               use_qk_l2norm_in_kernel, workspace=None, out=None, final_state=None,
               save_workspace=None, gate=None, name="chunk_gated_delta_rule"):
    """gdn_chunk_fwd, or gdn_chunk_fwd_save into ``save_workspace`` (a
    backward-sized workspace the backward then reuses), or with ``gate``
    gdn_chunk_fwd_gating (g, beta are then the gating inputs a, b)."""
    q, k, v, g, beta, cu, (B, T, Hqk, Hv, K, V, N) = _check_inputs(
        q, k, v, g, beta, initial_state, cu_seqlens, name, convert_gates=gate is None)
    if scale is None:
        scale = K ** -0.5
    dev = q.device
    o = torch.empty_like(v) if out is None else out
    if o.shape != v.shape or o.dtype != torch.bfloat16 or o.device != dev or not o.is_contiguous():
        raise ValueError(f"{name}: out must be a contiguous bf16 tensor of shape {tuple(v.shape)}.")
    h0 = initial_state.contiguous() if initial_state is not None else None
    ht = None
    if output_final_state:
        if final_state is None:
            ht = torch.empty((N, Hv, K, V), dtype=torch.float32, device=dev)
        else:
            ht = final_state
            if (tuple(ht.shape) != (N, Hv, K, V) or ht.dtype != torch.float32
                    or ht.device != dev or not ht.is_contiguous()):
                raise ValueError(f"{name}: final_state must be contiguous fp32 {(N, Hv, K, V)}.")
    entry = _native.lib().gdn_chunk_fwd
    if save_workspace is not None:
        workspace, entry = save_workspace, _native.lib().gdn_chunk_fwd_save
        nbytes = chunk_bwd_workspace_bytes(B, T, Hqk, Hv, K, V, N, cu is not None,
                                           use_qk_l2norm_in_kernel)
    else:
        nbytes = chunk_workspace_bytes(B, T, Hqk, Hv, K, V, N, cu is not None,
                                       use_qk_l2norm_in_kernel)
    if workspace is None:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < nbytes or workspace.device != dev:
        raise ValueError(f"{name}: workspace must be >= {nbytes} bytes on {dev}.")
    if gate is not None:
        rc = _native.lib().gdn_chunk_fwd_gating(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), *_gate_ptrs(gate, g, beta, Hv, dev, name),
            _ptr(h0), _ptr(ht), o.data_ptr(), _ptr(cu),
            B, T, Hqk, Hv, K, V, N, float(scale), int(bool(use_qk_l2norm_in_kernel)),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            _stream_ptr(dev))
        _native.check(rc, name)
        return o, ht
    rc = entry(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
        _ptr(h0), _ptr(ht), o.data_ptr(), _ptr(cu),
        B, T, Hqk, Hv, K, V, N, float(scale), int(bool(use_qk_l2norm_in_kernel)),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        _stream_ptr(dev))
    _native.check(rc, name)
    return o, ht


def fused_recurrent_gated_delta_rule(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    inplace_final_state: bool = True,
    ssm_state_indices: Optional[torch.Tensor] = None,
    num_accepted_tokens: Optional[torch.Tensor] = None,
    *,
    out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Token-by-token gated delta rule (decode) on gfx950.

    Semantics of torch_recurrent_gated_delta_rule (modeling_qwen3_next.py:
    456-503).  Each (sequence, v-head) state tile is read from HBM once,
    advanced through that sequence's tokens and written once.  With
    ``output_final_state`` and ``inplace_final_state`` (and an
    ``initial_state``) the final state overwrites ``initial_state`` and that
    tensor is returned; otherwise a new tensor is returned.

    Continuous batching: with ``ssm_state_indices`` (int32 [N]) the
    ``initial_state`` is a pool ``[num_slots, Hv, K, V]`` and sequence n
    reads slot ``ssm_state_indices[n]``; with ``output_final_state`` the
    slot is updated in place and the pool returned.  A slot outside
    ``[0, num_slots)`` marks a padding sequence: its state is untouched and
    its output rows are left unwritten.  Sequences must use distinct slots.

    Speculative decoding: with a 2-D ``ssm_state_indices`` (int32 [N, S]) the
    state after token t of sequence n is written to slot
    ``ssm_state_indices[n, t]`` (t < S; an entry outside the pool skips that
    write), so the states after every draft token are kept and a rejected
    draft is rolled back by starting the next step from the slot of the last
    accepted token: ``num_accepted_tokens`` (int32 [N]) selects the initial
    slot ``ssm_state_indices[n, num_accepted_tokens[n] - 1]`` (default entry
    0).  The pool is updated in place and returned.
    """
    name = "fused_recurrent_gated_delta_rule"
    if ssm_state_indices is not None and ssm_state_indices.dim() == 2:
        return _recurrent_spec(q, k, v, g, beta, scale, initial_state, cu_seqlens,
                               use_qk_l2norm_in_kernel, inplace_final_state, ssm_state_indices,
                               num_accepted_tokens, out, name)
    if num_accepted_tokens is not None:
        raise ValueError(f"{name}: num_accepted_tokens requires a 2-D ssm_state_indices [N, S].")
    if ssm_state_indices is not None:
        return _recurrent_indexed(q, k, v, g, beta, scale, initial_state, output_final_state,
                                  cu_seqlens, use_qk_l2norm_in_kernel, inplace_final_state,
                                  ssm_state_indices, out, name)
    return _recurrent_plain(q, k, v, g, beta, scale, initial_state, output_final_state,
                            cu_seqlens, use_qk_l2norm_in_kernel, inplace_final_state, out, name)


def _recurrent_plain(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
                     use_qk_l2norm_in_kernel, inplace_final_state, out, name, gate=None):
    q, k, v, g, beta, cu, (B, T, Hqk, Hv, K, V, N) = _check_inputs(
        q, k, v, g, beta, initial_state, cu_seqlens, name, convert_gates=gate is None)
    if scale is None:
        scale = K ** -0.5
    dev = q.device
    o = torch.empty_like(v) if out is None else out
    if o.shape != v.shape or o.dtype != torch.bfloat16 or o.device != dev or not o.is_contiguous():
        raise ValueError(f"{name}: out must be a contiguous bf16 tensor of shape {tuple(v.shape)}.")
    h0 = initial_state
    if h0 is not None and not h0.is_contiguous():
        if output_final_state and inplace_final_state:
            raise ValueError(f"{name}: an in-place initial_state must be contiguous.")
        h0 = h0.contiguous()
    ht = None
    if output_final_state:
        if inplace_final_state and h0 is not None:
            ht = h0
        else:
            ht = torch.empty((N, Hv, K, V), dtype=torch.float32, device=dev)
    if gate is not None:
        rc = _native.lib().gdn_recurrent_fwd_gating(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), *_gate_ptrs(gate, g, beta, Hv, dev, name),
            _ptr(h0), _ptr(ht), o.data_ptr(), _ptr(cu), None,
            B, T, Hqk, Hv, K, V, N, N, float(scale), int(bool(use_qk_l2norm_in_kernel)),
            _stream_ptr(dev))
    else:
        rc = _native.lib().gdn_recurrent_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
            _ptr(h0), _ptr(ht), o.data_ptr(), _ptr(cu),
            B, T, Hqk, Hv, K, V, N, float(scale), int(bool(use_qk_l2norm_in_kernel)),
            _stream_ptr(dev))
    _native.check(rc, name)
    return o, ht


def _recurrent_indexed(q, k, v, g, beta, scale, pool, output_final_state, cu_seqlens,
                       use_qk_l2norm_in_kernel, inplace_final_state, idx, out, name, gate=None):
    if pool is None or not isinstance(pool, torch.Tensor) or pool.dim() != 4:
        raise ValueError(f"{name}: ssm_state_indices requires initial_state as a state pool "
                         "[num_slots, Hv, K, V].")
    if output_final_state and not inplace_final_state:
        raise ValueError(f"{name}: with ssm_state_indices the final state is written in place.")
    q, k, v, g, beta, cu, (B, T, Hqk, Hv, K, V, N) = _check_inputs(
        q, k, v, g, beta, None, cu_seqlens, name, convert_gates=gate is None)
    dev = q.device
    if (tuple(pool.shape[1:]) != (Hv, K, V) or pool.dtype != torch.float32
            or pool.device != dev or not pool.is_contiguous()):
        raise ValueError(f"{name}: the state pool must be a contiguous fp32 tensor "
                         f"[num_slots, {Hv}, {K}, {V}] on {dev}.")
    if (not isinstance(idx, torch.Tensor) or tuple(idx.shape) != (N,)
            or idx.dtype != torch.int32 or idx.device not in (dev, torch.device("cpu"))):
        raise ValueError(f"{name}: ssm_state_indices must be int32 of shape ({N},) on {dev} "
                         "or the CPU.")
    _check_distinct_slots(idx, pool.shape[0], name)
    idx = idx.to(dev)
    if scale is None:
        scale = K ** -0.5
    o = torch.empty_like(v) if out is None else out
    if o.shape != v.shape or o.dtype != torch.bfloat16 or o.device != dev or not o.is_contiguous():
        raise ValueError(f"{name}: out must be a contiguous bf16 tensor of shape {tuple(v.shape)}.")
    ht = pool if output_final_state else None
    if gate is not None:
        rc = _native.lib().gdn_recurrent_fwd_gating(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), *_gate_ptrs(gate, g, beta, Hv, dev, name),
            pool.data_ptr(), _ptr(ht), o.data_ptr(), _ptr(cu), idx.contiguous().data_ptr(),
            B, T, Hqk, Hv, K, V, N, pool.shape[0], float(scale),
            int(bool(use_qk_l2norm_in_kernel)), _stream_ptr(dev))
    else:
        rc = _native.lib().gdn_recurrent_fwd_indexed(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
            pool.data_ptr(), _ptr(ht), o.data_ptr(), _ptr(cu), idx.contiguous().data_ptr(),
            B, T, Hqk, Hv, K, V, N, pool.shape[0], float(scale),
            int(bool(use_qk_l2norm_in_kernel)), _stream_ptr(dev))
    _native.check(rc, name)
    return o, ht


def _check_distinct_slots(idx: torch.Tensor, num_slots: int, name: str) -> None:
    """Reject a host-resident slot table that gives two sequences (rows) the
    same slot, before anything is launched.  A device-resident table is
    checked by the kernel itself: every sequence involved leaves its slots
    untouched and gets NaN output rows."""
    if idx.device.type != "cpu":
        return
    if idx.numel() == 0:
        return
    rows = idx.reshape(idx.shape[0], -1) if idx.dim() else idx.reshape(1, 1)
    seen = torch.cat([torch.unique(r[(r >= 0) & (r < num_slots)]) for r in rows])
    if seen.numel() != torch.unique(seen).numel():
        raise ValueError(f"{name}: ssm_state_indices gives two sequences the same slot.")


def _recurrent_spec(q, k, v, g, beta, scale, pool, cu_seqlens, use_qk_l2norm_in_kernel,
                    inplace_final_state, idx, accepted, out, name):
    if pool is None or not isinstance(pool, torch.Tensor) or pool.dim() != 4:
        raise ValueError(f"{name}: a 2-D ssm_state_indices requires initial_state as a state "
                         "pool [num_slots, Hv, K, V].")
    if not inplace_final_state:
        raise ValueError(f"{name}: with ssm_state_indices the states are written in place.")
    q, k, v, g, beta, cu, (B, T, Hqk, Hv, K, V, N) = _check_inputs(
        q, k, v, g, beta, None, cu_seqlens, name)
    dev = q.device
    if (tuple(pool.shape[1:]) != (Hv, K, V) or pool.dtype != torch.float32
            or pool.device != dev or not pool.is_contiguous()):
        raise ValueError(f"{name}: the state pool must be a contiguous fp32 tensor "
                         f"[num_slots, {Hv}, {K}, {V}] on {dev}.")
    if (not isinstance(idx, torch.Tensor) or idx.dim() != 2 or idx.shape[0] != N
            or idx.dtype != torch.int32):
        raise ValueError(f"{name}: a 2-D ssm_state_indices must be int32 of shape ({N}, S).")
    if cu is None and T > idx.shape[1]:
        raise ValueError(f"{name}: T ({T}) exceeds the ssm_state_indices row length "
                         f"({idx.shape[1]}).")
    _check_distinct_slots(idx, pool.shape[0], name)
    idx = idx.to(dev).contiguous()
    if accepted is not None:
        if (not isinstance(accepted, torch.Tensor) or tuple(accepted.shape) != (N,)
                or accepted.dtype != torch.int32):
            raise ValueError(f"{name}: num_accepted_tokens must be int32 of shape ({N},).")
        accepted = accepted.to(dev).contiguous()
    if scale is None:
        scale = K ** -0.5
    o = torch.empty_like(v) if out is None else out
    if o.shape != v.shape or o.dtype != torch.bfloat16 or o.device != dev or not o.is_contiguous():
        raise ValueError(f"{name}: out must be a contiguous bf16 tensor of shape {tuple(v.shape)}.")
    rc = _native.lib().gdn_recurrent_fwd_spec(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
        pool.data_ptr(), o.data_ptr(), _ptr(cu), idx.data_ptr(), idx.shape[1], _ptr(accepted),
        B, T, Hqk, Hv, K, V, N, pool.shape[0], float(scale),
        int(bool(use_qk_l2norm_in_kernel)), _stream_ptr(dev))
    _native.check(rc, name)
    return o, pool


# ------------------------------------------------ gating fused into the core
def _gate_ptrs(gate, a, b, Hv, dev, name):
    """Pointer / code arguments of the *_gating entry points, after checking
    A_log, dt_bias ([Hv], one dtype) and the gating inputs a, b."""
    from .layer_ops import _dt
    A_log, dt_bias, spb, spt = gate
    for nm, t in (("A_log", A_log), ("dt_bias", dt_bias)):
        if not isinstance(t, torch.Tensor) or tuple(t.shape) != (Hv,) or t.device != dev:
            raise ValueError(f"{name}: {nm} must be a tensor of shape ({Hv},) on {dev}.")
    if A_log.dtype != dt_bias.dtype:
        raise ValueError(f"{name}: A_log and dt_bias must share a dtype.")
    if not spb > 0:
        raise ValueError(f"{name}: softplus beta must be > 0.")
    adt, bdt, pdt = _dt(a, name, "a"), _dt(b, name, "b"), _dt(A_log, name, "A_log")
    return (A_log.contiguous().data_ptr(), a.data_ptr(), b.data_ptr(),
            dt_bias.contiguous().data_ptr(), adt, bdt, pdt, float(spb), float(spt))


def chunk_gated_delta_rule_gated(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    softplus_beta: float = 1.0,
    softplus_threshold: float = 20.0,
    *,
    workspace: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    save_for_backward: Optional[bool] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """``chunk_gated_delta_rule`` with the layer's gating fused in.

    The Qwen3-Next layer forms ``g = -exp(A_log) * softplus(a + dt_bias)``
    and ``beta = sigmoid(b)`` (modeling_qwen3_next.py:650-652) and passes
    them to the core (:672-683).  Here the core's prep kernel forms them
    itself from ``a``, ``b`` ([B, T, Hv], bf16 / fp16 / fp32) and ``A_log``,
    ``dt_bias`` ([Hv]) -- the same definition as ``fused_gdn_gating``, so the
    result equals ``chunk_gated_delta_rule(q, k, v, *fused_gdn_gating(...))``
    bit for bit -- and no fp32 g / beta tensor exists.

    Differentiable: when any of q, k, v, a, b, A_log, dt_bias, initial_state
    requires grad (and grad mode is on) the call is exactly that composition
    under autograd -- ``fused_gdn_gating`` (its backward one kernel,
    ``fused_gdn_gating_bwd``: da, db and the per-head sums of dA_log and
    ddt_bias) feeding ``chunk_gated_delta_rule`` (backward gdn_chunk_bwd);
    g and beta (fp32, 4 bytes per token and v-head each) are then held for
    the backward.  ``save_for_backward`` as for ``chunk_gated_delta_rule``.
    """
    if torch.is_grad_enabled() and any(
            isinstance(t, torch.Tensor) and t.requires_grad
            for t in (q, k, v, a, b, A_log, dt_bias, initial_state)):
        if out is not None or workspace is not None:
            raise ValueError("chunk_gated_delta_rule_gated: out / workspace buffers are not "
                             "supported when gradients are required.")
        g, beta = fused_gdn_gating(A_log, a, b, dt_bias, softplus_beta, softplus_threshold)
        return chunk_gated_delta_rule(q, k, v, g, beta, scale, initial_state,
                                      output_final_state, cu_seqlens, use_qk_l2norm_in_kernel,
                                      save_for_backward=save_for_backward)
    return _chunk_fwd(q, k, v, a, b, scale, initial_state, output_final_state, cu_seqlens,
                      use_qk_l2norm_in_kernel, workspace=workspace, out=out,
                      gate=(A_log, dt_bias, softplus_beta, softplus_threshold),
                      name="chunk_gated_delta_rule_gated")


def fused_recurrent_gated_delta_rule_gated(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    inplace_final_state: bool = True,
    ssm_state_indices: Optional[torch.Tensor] = None,
    softplus_beta: float = 1.0,
    softplus_threshold: float = 20.0,
    *,
    out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """``fused_recurrent_gated_delta_rule`` (plain, or over a slot pool with a
    1-D ``ssm_state_indices``) with the layer's gating fused in: the decode
    kernel forms g and beta from ``a``, ``b``, ``A_log``, ``dt_bias`` per
    token (see ``chunk_gated_delta_rule_gated``)."""
    name = "fused_recurrent_gated_delta_rule_gated"
    gate = (A_log, dt_bias, softplus_beta, softplus_threshold)
    if ssm_state_indices is not None:
        if ssm_state_indices.dim() != 1:
            raise ValueError(f"{name}: ssm_state_indices must be 1-D [N].")
        return _recurrent_indexed(q, k, v, a, b, scale, initial_state, output_final_state,
                                  cu_seqlens, use_qk_l2norm_in_kernel, inplace_final_state,
                                  ssm_state_indices, out, name, gate=gate)
    return _recurrent_plain(q, k, v, a, b, scale, initial_state, output_final_state, cu_seqlens,
                            use_qk_l2norm_in_kernel, inplace_final_state, out, name, gate=gate)
