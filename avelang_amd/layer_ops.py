"""Producer / consumer operators of a Qwen3-Next linear-attention layer on gfx950.

The gated-delta-net core (``gated_delta_rule.py``) consumes q/k/v from a
causal depthwise convolution, decay / write gates computed from two small
projections, and L2-normalised q/k; its output goes through a gated
RMSNorm.  These operators are those neighbours, with the argument lists of
the kernel libraries the layer binds to:

    fused_gdn_gating        g, beta from (A_log, a, b, dt_bias)     TF:650-652
                            (differentiable: fused_gdn_gating_bwd)
    l2norm_fwd              row L2 normalisation                     TF:368-371
    causal_conv1d_fn        prefill convolution (+ SiLU)             TF:346-365
    causal_conv1d_update    decode convolution, state in place       TF:326-343
    rms_norm_gated          gated RMSNorm (norm before gate)         TF:58-74, :693

(TF = transformers 5.15.0 models/qwen3_next/modeling_qwen3_next.py, read as
text.)  The reference repository has no counterpart; the wrappers follow its
kernel-library convention (python/avelang_kernels/amdgpu_gemm.py:458-494):
``ValueError`` before any launch, outputs allocated on the input's device,
asynchronous launch on torch's current stream.  Every operator calls the
HIP kernels of ``csrc/gdn_layer.hip`` through ``include/gdn_layer.h``; there
is no fallback path.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from . import _native

__all__ = [
    "fused_gdn_gating",
    "fused_gdn_gating_bwd",
    "l2norm_fwd",
    "causal_conv1d_fn",
    "causal_conv1d_update",
    "rms_norm_gated",
]

_DTYPES = {
    torch.float32: _native.GDN_DTYPE_F32,
    torch.bfloat16: _native.GDN_DTYPE_BF16,
    torch.float16: _native.GDN_DTYPE_F16,
}


def _dt(t: torch.Tensor, name: str, what: str) -> int:
    if t.dtype not in _DTYPES:
        raise ValueError(f"{name}: {what} must be float32, bfloat16 or float16, got {t.dtype}.")
    return _DTYPES[t.dtype]


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _on(dev: torch.device, name: str, **tensors) -> None:
    if dev.type != "cuda":
        raise ValueError(f"{name}: tensors must be on a ROCm (cuda) device, got {dev}.")
    for nm, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name}: {nm} must be on {dev}, got {t.device}.")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the row kernels move 16 bytes per lane)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _silu_flag(activation: Optional[str], name: str) -> int:
    if activation is None:
        return 0
    if activation in ("silu", "swish"):
        return 1
    raise ValueError(f"{name}: activation must be None, 'silu' or 'swish', got {activation!r}.")


def fused_gdn_gating(
    A_log: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    dt_bias: torch.Tensor,
    beta: float = 1.0,
    threshold: float = 20.0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Decay and write-strength gates of the layer (TF:650-652).

    ``g = -exp(A_log) * softplus(a + dt_bias)`` and ``beta = sigmoid(b)``,
    computed in fp32 and returned as fp32 tensors with ``a``'s shape (the
    head axis last).  ``beta`` / ``threshold`` are softplus's parameters.
    The layer text evaluates ``b.sigmoid()`` in ``b``'s own dtype; here it
    is kept in fp32 (a difference below one bf16 ulp of beta).

    Differentiable: when any input requires grad (and grad mode is on) the
    backward is ``fused_gdn_gating_bwd`` (one kernel for da, db and the
    per-head sums of dA_log and ddt_bias).
    """
    if torch.is_grad_enabled() and any(
            isinstance(t, torch.Tensor) and t.requires_grad for t in (A_log, a, b, dt_bias)):
        return _GdnGating.apply(A_log, a, b, dt_bias, float(beta), float(threshold))
    return _gating_fwd(A_log, a, b, dt_bias, beta, threshold)


def _gating_args(A_log, a, b, dt_bias, beta, name):
    """Validated, contiguous (A_log, a, b, dt_bias) and their dtype codes."""
    for nm, t in (("A_log", A_log), ("a", a), ("b", b), ("dt_bias", dt_bias)):
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"{name}: {nm} must be a torch.Tensor")
    if a.dim() < 1 or a.shape != b.shape:
        raise ValueError(f"{name}: a and b must have the same shape [..., H], got "
                         f"{tuple(a.shape)} and {tuple(b.shape)}.")
    H = a.shape[-1]
    if H == 0 or tuple(A_log.shape) != (H,) or tuple(dt_bias.shape) != (H,):
        raise ValueError(f"{name}: A_log and dt_bias must have shape ({H},).")
    if A_log.dtype != dt_bias.dtype:
        raise ValueError(f"{name}: A_log and dt_bias must share a dtype.")
    if not beta > 0:
        raise ValueError(f"{name}: softplus beta must be > 0.")
    adt, bdt, pdt = _dt(a, name, "a"), _dt(b, name, "b"), _dt(A_log, name, "A_log")
    _on(a.device, name, b=b, A_log=A_log, dt_bias=dt_bias)
    a, b, A_log, dt_bias = (t.contiguous() for t in (a, b, A_log, dt_bias))
    return A_log, a, b, dt_bias, adt, bdt, pdt


def _gating_fwd(A_log, a, b, dt_bias, beta, threshold):
    name = "fused_gdn_gating"
    A_log, a, b, dt_bias, adt, bdt, pdt = _gating_args(A_log, a, b, dt_bias, beta, name)
    H = a.shape[-1]
    dev = a.device
    g = torch.empty(a.shape, dtype=torch.float32, device=dev)
    beta_out = torch.empty(a.shape, dtype=torch.float32, device=dev)
    rows = a.numel() // H
    rc = _native.lib().gdn_gating_fwd(
        A_log.data_ptr(), a.data_ptr(), b.data_ptr(), dt_bias.data_ptr(), g.data_ptr(),
        beta_out.data_ptr(), rows, H, adt, bdt, pdt, float(beta), float(threshold), _stream(dev))
    _native.check(rc, name)
    return g, beta_out


def fused_gdn_gating_bwd(
    A_log: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    dt_bias: torch.Tensor,
    dg: torch.Tensor,
    dbeta: Optional[torch.Tensor] = None,
    beta: float = 1.0,
    threshold: float = 20.0,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], torch.Tensor]:
    """Gradients of ``fused_gdn_gating`` (autograd of TF:650-652) given
    ``dg`` / ``dbeta`` (``a``'s shape): ``(dA_log, da, db, ddt_bias)``.

    ``da = dg * -exp(A_log) * softplus'(a + dt_bias)`` and ``db = dbeta *
    beta * (1 - beta)`` in ``a``'s / ``b``'s dtype; ``ddt_bias`` (the fp32
    sum of da over every leading axis) and ``dA_log`` (that of ``dg * g``)
    in the parameters' dtype, summed in a fixed order (deterministic).
    ``softplus'`` is torch's: ``sigmoid(beta x)``, 1 above the threshold.
    ``db`` is None when ``dbeta`` is.
    """
    name = "fused_gdn_gating_bwd"
    A_log, a, b, dt_bias, adt, bdt, pdt = _gating_args(A_log, a, b, dt_bias, beta, name)
    H = a.shape[-1]
    dev = a.device
    for nm, t in (("dg", dg), ("dbeta", dbeta)):
        if t is not None and (not isinstance(t, torch.Tensor) or t.shape != a.shape
                              or t.device != dev):
            raise ValueError(f"{name}: {nm} must be a tensor of shape {tuple(a.shape)} on {dev}.")
    dg = dg.float().contiguous()
    dbeta = dbeta.float().contiguous() if dbeta is not None else None
    rows = a.numel() // H
    da = torch.empty_like(a)
    db = torch.empty_like(b) if dbeta is not None else None
    dA_log = torch.empty_like(A_log)
    ddt = torch.empty_like(dt_bias)
    lib = _native.lib()
    nbytes = lib.gdn_gating_bwd_workspace_bytes(rows, H)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    rc = lib.gdn_gating_bwd(
        A_log.data_ptr(), a.data_ptr(), b.data_ptr(), dt_bias.data_ptr(), dg.data_ptr(),
        _ptr(dbeta), dA_log.data_ptr(), da.data_ptr(), _ptr(db), ddt.data_ptr(), rows, H,
        adt, bdt, pdt, float(beta), float(threshold), ws.data_ptr(), nbytes, _stream(dev))
    _native.check(rc, name)
    return dA_log, da, db, ddt


class _GdnGating(torch.autograd.Function):
    """Autograd form of fused_gdn_gating: forward gdn_gating_fwd, backward
    gdn_gating_bwd."""

    @staticmethod
    def forward(ctx, A_log, a, b, dt_bias, beta, threshold):
        g, beta_out = _gating_fwd(A_log, a, b, dt_bias, beta, threshold)
        ctx.save_for_backward(A_log, a, b, dt_bias)
        ctx.sp = (beta, threshold)
        return g, beta_out

    @staticmethod
    def backward(ctx, dg, dbeta):
        A_log, a, b, dt_bias = ctx.saved_tensors
        if dg is None:
            dg = torch.zeros(a.shape, dtype=torch.float32, device=a.device)
        dA_log, da, db, ddt = fused_gdn_gating_bwd(A_log, a, b, dt_bias, dg, dbeta, *ctx.sp)
        if db is None:
            db = torch.zeros_like(b)
        return dA_log, da, db, ddt, None, None


def l2norm_fwd(x: torch.Tensor, eps: float = 1e-6,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x * rsqrt(sum(x^2, -1) + eps)`` over the last axis (TF:368-371).

    fp32 arithmetic, result in ``x``'s dtype; last axis of 64, 128 or 256.
    ``out`` may be ``x`` itself.
    """
    name = "l2norm_fwd"
    if not isinstance(x, torch.Tensor) or x.dim() < 1:
        raise ValueError(f"{name}: x must be a tensor with at least one axis.")
    D = x.shape[-1]
    if D not in (64, 128, 256):
        raise ValueError(f"{name}: last axis must be 64, 128 or 256, got {D}.")
    dt = _dt(x, name, "x")
    dev = x.device
    _on(dev, name, out=out)
    x = _aligned(x)
    y = torch.empty_like(x) if out is None else out
    if (y.shape != x.shape or y.dtype != x.dtype or not y.is_contiguous()
            or y.data_ptr() % 16):
        raise ValueError(f"{name}: out must be a contiguous, 16-byte aligned {x.dtype} tensor "
                         f"of shape {tuple(x.shape)}.")
    rc = _native.lib().gdn_l2norm_fwd(x.data_ptr(), y.data_ptr(), x.numel() // D, D,
                                      float(eps), dt, _stream(dev))
    _native.check(rc, name)
    return y


def causal_conv1d_fn(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    seq_idx: Optional[torch.Tensor] = None,
    initial_states: Optional[torch.Tensor] = None,
    return_final_states: bool = False,
    final_states_out: Optional[torch.Tensor] = None,
    activation: Optional[str] = None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Causal depthwise convolution over time (TF:346-365).

    ``x [B, D, T]`` with any strides: the layer's channel-last memory (a
    ``[B, T, D]`` tensor viewed as ``[B, D, T]``) and time-contiguous
    ``[B, D, T]`` take vectorised kernels.  ``weight [D, W]`` (W in 2..4),
    ``bias [D]``; ``activation`` None or "silu"/"swish".  ``seq_idx [B, T]``
    int32 keeps packed sequences apart; ``initial_states [B, D, W-1]`` are
    the inputs before t = 0; with ``return_final_states`` the last W-1
    inputs of each row are returned too (into ``final_states_out`` if
    given).  The output has ``x``'s layout and dtype.
    """
    name = "causal_conv1d_fn"
    if not isinstance(x, torch.Tensor) or x.dim() != 3:
        raise ValueError(f"{name}: x must be a 3-D tensor [B, D, T].")
    B, D, T = x.shape
    if not isinstance(weight, torch.Tensor) or weight.dim() != 2 or weight.shape[0] != D:
        raise ValueError(f"{name}: weight must have shape ({D}, W).")
    W = weight.shape[1]
    if W not in (2, 3, 4):
        raise ValueError(f"{name}: kernel width must be 2, 3 or 4, got {W}.")
    if bias is not None and (tuple(bias.shape) != (D,) or bias.dtype != weight.dtype):
        raise ValueError(f"{name}: bias must have shape ({D},) and weight's dtype.")
    dt, wdt = _dt(x, name, "x"), _dt(weight, name, "weight")
    silu = _silu_flag(activation, name)
    dev = x.device
    _on(dev, name, weight=weight, bias=bias, seq_idx=seq_idx, initial_states=initial_states,
        final_states_out=final_states_out)
    if seq_idx is not None:
        if tuple(seq_idx.shape) != (B, T) or seq_idx.dtype != torch.int32:
            raise ValueError(f"{name}: seq_idx must be int32 of shape ({B}, {T}).")
        if initial_states is not None:
            raise ValueError(f"{name}: seq_idx and initial_states cannot be combined.")
        seq_idx = seq_idx.contiguous()
    if initial_states is not None:
        if tuple(initial_states.shape) != (B, D, W - 1) or initial_states.dtype != x.dtype:
            raise ValueError(f"{name}: initial_states must be {x.dtype} of shape ({B}, {D}, {W - 1}).")
        initial_states = initial_states.contiguous()
    fin = None
    if return_final_states:
        fin = final_states_out
        if fin is None:
            fin = torch.empty((B, D, W - 1), dtype=x.dtype, device=dev)
        elif (tuple(fin.shape) != (B, D, W - 1) or fin.dtype != x.dtype
              or not fin.is_contiguous()):
            raise ValueError(f"{name}: final_states_out must be contiguous {x.dtype} ({B}, {D}, {W - 1}).")
    weight = weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    out = torch.empty_like(x)
    sx, so = x.stride(), out.stride()
    rc = _native.lib().gdn_causal_conv1d_fwd(
        x.data_ptr(), weight.data_ptr(), _ptr(bias), _ptr(seq_idx), _ptr(initial_states),
        _ptr(fin), out.data_ptr(), B, D, T, W, sx[0], sx[1], sx[2], so[0], so[1], so[2],
        silu, dt, wdt, _stream(dev))
    _native.check(rc, name)
    return (out, fin) if return_final_states else out


def causal_conv1d_update(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    activation: Optional[str] = None,
    conv_state_indices: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Decode step of the convolution with ``conv_state`` updated in place
    (TF:326-343).

    ``x [B, D]`` or ``[B, D, L]`` (L <= 64 new tokens per row);
    ``conv_state [num_slots, D, S]`` contiguous in ``x``'s dtype, W-1 <= S <= 8;
    row b uses slot ``conv_state_indices[b]`` (int32 [B]; b when None), and a
    slot outside ``[0, num_slots)`` marks a padding row that is skipped
    (its output is left unwritten).  Rows must map to distinct slots.
    Returns the output with ``x``'s shape and dtype.
    """
    name = "causal_conv1d_update"
    if not isinstance(x, torch.Tensor) or x.dim() not in (2, 3):
        raise ValueError(f"{name}: x must be [B, D] or [B, D, L].")
    squeeze = x.dim() == 2
    x3 = x.unsqueeze(-1) if squeeze else x
    B, D, L = x3.shape
    if not isinstance(weight, torch.Tensor) or weight.dim() != 2 or weight.shape[0] != D:
        raise ValueError(f"{name}: weight must have shape ({D}, W).")
    W = weight.shape[1]
    if W not in (2, 3, 4):
        raise ValueError(f"{name}: kernel width must be 2, 3 or 4, got {W}.")
    if not 1 <= L <= 64:
        raise ValueError(f"{name}: 1 <= L <= 64 new tokens per row, got {L}.")
    if (not isinstance(conv_state, torch.Tensor) or conv_state.dim() != 3
            or conv_state.shape[1] != D or conv_state.dtype != x.dtype
            or not conv_state.is_contiguous()):
        raise ValueError(f"{name}: conv_state must be a contiguous {x.dtype} tensor [slots, {D}, S].")
    S = conv_state.shape[2]
    if not W - 1 <= S <= 8:
        raise ValueError(f"{name}: conv_state length must be in [{W - 1}, 8], got {S}.")
    if bias is not None and (tuple(bias.shape) != (D,) or bias.dtype != weight.dtype):
        raise ValueError(f"{name}: bias must have shape ({D},) and weight's dtype.")
    dt, wdt = _dt(x, name, "x"), _dt(weight, name, "weight")
    silu = _silu_flag(activation, name)
    dev = x.device
    _on(dev, name, conv_state=conv_state, weight=weight, bias=bias,
        conv_state_indices=conv_state_indices)
    num_slots = conv_state.shape[0]
    if conv_state_indices is not None:
        if tuple(conv_state_indices.shape) != (B,) or conv_state_indices.dtype != torch.int32:
            raise ValueError(f"{name}: conv_state_indices must be int32 of shape ({B},).")
        conv_state_indices = conv_state_indices.contiguous()
    elif num_slots < B:
        raise ValueError(f"{name}: conv_state has {num_slots} slots for {B} rows.")
    weight = weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    out = torch.empty_like(x3)
    sx, so = x3.stride(), out.stride()
    rc = _native.lib().gdn_causal_conv1d_update(
        x3.data_ptr(), conv_state.data_ptr(), weight.data_ptr(), _ptr(bias),
        _ptr(conv_state_indices), out.data_ptr(), B, D, L, W, S, num_slots,
        sx[0], sx[1], sx[2], so[0], so[1], so[2], silu, dt, wdt, _stream(dev))
    _native.check(rc, name)
    return out.squeeze(-1) if squeeze else out


def rms_norm_gated(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor,
                   eps: float = 1e-6) -> torch.Tensor:
    """Gated RMSNorm of the layer, norm before gate (TF:58-74, used at :693).

    ``x``, ``z`` of the same shape ``[..., D]`` (D in 64/128/256) and dtype,
    ``weight [D]``.  Rounding follows the layer: the normalised value is
    rounded to ``x``'s dtype, multiplied by ``weight`` (rounded again when
    ``weight`` has ``x``'s dtype), times ``silu(z)`` in fp32, rounded.
    """
    name = "rms_norm_gated"
    if not isinstance(x, torch.Tensor) or not isinstance(z, torch.Tensor) or x.dim() < 1:
        raise ValueError(f"{name}: x and z must be tensors.")
    if x.shape != z.shape or x.dtype != z.dtype:
        raise ValueError(f"{name}: z must match x's shape and dtype.")
    D = x.shape[-1]
    if D not in (64, 128, 256):
        raise ValueError(f"{name}: last axis must be 64, 128 or 256, got {D}.")
    if not isinstance(weight, torch.Tensor) or tuple(weight.shape) != (D,):
        raise ValueError(f"{name}: weight must have shape ({D},).")
    dt, wdt = _dt(x, name, "x"), _dt(weight, name, "weight")
    dev = x.device
    _on(dev, name, z=z, weight=weight)
    x, z, weight = _aligned(x), _aligned(z), weight.contiguous()
    out = torch.empty_like(x)
    rc = _native.lib().gdn_rmsnorm_gated_fwd(x.data_ptr(), z.data_ptr(), weight.data_ptr(),
                                             out.data_ptr(), x.numel() // D, D, float(eps), dt,
                                             wdt, _stream(dev))
    _native.check(rc, name)
    return out
