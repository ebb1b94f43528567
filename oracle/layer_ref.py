"""numpy oracle for the layer operators around the GDN core
(TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product never does.

Semantics follow transformers' Qwen3-Next layer text
(models/qwen3_next/modeling_qwen3_next.py, 5.15.0, read as text):
    gating                 :650-652   g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
    gating_bwd             autograd of :650-652 (torch's softplus backward)
    l2norm                 :368-371   (in gdn_ref)
    causal_conv1d          :346-365   depthwise conv over time, zero left padding, SiLU
    causal_conv1d_update   :326-343   conv over concat(state, x), state <- last S inputs
    rmsnorm_gated          :58-74     norm before gate, with the layer's roundings
and, for continuous batching, ``recurrent_indexed``: the per-token recurrence
of gdn_ref applied to slots of a state pool.  Pinning checks live in
tests/test_layer_oracle.py.
"""
from __future__ import annotations

import numpy as np

from . import gdn_ref

__all__ = [
    "bf16_round",
    "f16_round",
    "gating",
    "gating_bwd",
    "causal_conv1d",
    "causal_conv1d_update",
    "rmsnorm_gated",
    "recurrent_indexed",
]


def bf16_round(x):
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def f16_round(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def _rounder(kind):
    if kind in (None, "f32", np.float32):
        return lambda v: np.asarray(v, dtype=np.float32)
    if kind == "bf16":
        return bf16_round
    if kind == "f16":
        return f16_round
    raise ValueError(kind)


def gating(A_log, a, b, dt_bias, sp_beta=1.0, threshold=20.0):
    """(g, beta) in float64 from float64 copies of the inputs (head axis last)."""
    A_log = np.asarray(A_log, np.float64)
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    dt_bias = np.asarray(dt_bias, np.float64)
    x = a + dt_bias
    bx = sp_beta * x
    with np.errstate(over="ignore"):
        sp = np.where(bx > threshold, x, np.log1p(np.exp(np.minimum(bx, threshold))) / sp_beta)
    g = -np.exp(A_log) * sp
    beta = 1.0 / (1.0 + np.exp(-b))
    return g, beta


def gating_bwd(A_log, a, b, dt_bias, dg, dbeta, sp_beta=1.0, threshold=20.0):
    """Gradients of ``gating``'s (g, beta) w.r.t. (A_log, a, b, dt_bias) given
    dg, dbeta (a's shape, head axis last), float64: (dA_log, da, db, ddt_bias).

    d softplus(x) / dx = sigmoid(sp_beta x), or 1 where sp_beta x > threshold
    (torch.nn.functional.softplus's backward); dg/dA_log = g; the per-head
    parameters' gradients sum over every leading axis.
    """
    A_log, a, b, dt_bias, dg, dbeta = (np.asarray(t, np.float64)
                                       for t in (A_log, a, b, dt_bias, dg, dbeta))
    bx = sp_beta * (a + dt_bias)
    with np.errstate(over="ignore"):
        dsp = np.where(bx > threshold, 1.0, 1.0 / (1.0 + np.exp(-np.minimum(bx, threshold))))
    g, beta = gating(A_log, a, b, dt_bias, sp_beta, threshold)
    da = dg * -np.exp(A_log) * dsp
    db = dbeta * beta * (1.0 - beta)
    lead = tuple(range(a.ndim - 1))
    return (dg * g).sum(axis=lead), da, db, da.sum(axis=lead)


def causal_conv1d(x, weight, bias=None, seq_idx=None, initial_states=None, silu=False):
    """x [B, D, T] -> (out [B, D, T], final_states [B, D, W-1]) in float64.

    out[b, d, t] = act(bias[d] + sum_j w[d, j] x[b, d, t - (W-1) + j]); inputs
    before t = 0 come from initial_states (else 0); with seq_idx [B, T] a
    window position with a different sequence id than t contributes 0.
    """
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    B, D, T = x.shape
    W = w.shape[1]
    init = (np.zeros((B, D, W - 1)) if initial_states is None
            else np.asarray(initial_states, np.float64))
    xp = np.concatenate([init, x], axis=2)            # [B, D, W-1+T]
    out = np.zeros((B, D, T))
    for j in range(W):
        term = w[:, j][None, :, None] * xp[:, :, j:j + T]
        if seq_idx is not None:
            sq = np.asarray(seq_idx)
            pos = np.arange(T) - (W - 1) + j           # window position per t
            valid = pos >= 0
            same = np.zeros((B, T), bool)
            same[:, valid] = sq[:, pos[valid]] == sq[:, valid]
            term = term * same[:, None, :]
        out += term
    if bias is not None:
        out += np.asarray(bias, np.float64)[None, :, None]
    if silu:
        out = out / (1.0 + np.exp(-out))
    final = xp[:, :, xp.shape[2] - (W - 1):]
    return out, final


def causal_conv1d_update(x, conv_state, weight, bias=None, indices=None, silu=False):
    """x [B, D, L], conv_state [slots, D, S] -> (out [B, D, L], new conv_state) in float64.

    Row b uses slot indices[b] (b when None); slots outside the pool are
    padding rows whose output stays NaN here and whose state is untouched.
    """
    x = np.asarray(x, np.float64)
    state = np.array(conv_state, np.float64, copy=True)
    w = np.asarray(weight, np.float64)
    B, D, L = x.shape
    S = state.shape[2]
    W = w.shape[1]
    out = np.full((B, D, L), np.nan)
    for bi in range(B):
        slot = bi if indices is None else int(indices[bi])
        if slot < 0 or slot >= state.shape[0]:
            continue
        win = np.concatenate([state[slot], x[bi]], axis=1)     # [D, S+L]
        for t in range(L):
            seg = win[:, S + t - (W - 1):S + t + 1]
            o = (seg * w).sum(1)
            if bias is not None:
                o = o + np.asarray(bias, np.float64)
            out[bi, :, t] = o / (1.0 + np.exp(-o)) if silu else o
        state[slot] = win[:, L:L + S]
    return out, state


def rmsnorm_gated(x, z, weight, eps=1e-6, dtype="f32", weight_dtype="f32"):
    """Gated RMSNorm, norm before gate, with the layer's rounding steps.

    n = round(x * rsqrt(mean(x^2) + eps)); wn = weight * n, rounded when the
    weight has the input's type; out = round(wn * silu(z)).  Computation in
    float32 like the layer (x and z are upcast to fp32).
    """
    rnd = _rounder(dtype)
    x = np.asarray(x, np.float32)
    z = np.asarray(z, np.float32)
    w = np.asarray(weight, np.float32)
    var = (x.astype(np.float64) ** 2).mean(-1, keepdims=True)
    n = rnd(x * (1.0 / np.sqrt(var + eps)).astype(np.float32))
    wn = w * n
    if weight_dtype == dtype:
        wn = rnd(wn)
    sz = z / (np.float32(1.0) + np.exp(-z))
    return rnd(wn * sz)


def recurrent_indexed(q, k, v, g, beta, pool, indices, scale=None, cu_seqlens=None,
                      use_qk_l2norm=False, dtype=np.float64):
    """Per-token recurrence over state slots: sequence n advances pool[indices[n]].

    Returns (o with padding sequences' rows NaN, new pool).
    """
    pool = np.array(pool, dtype=dtype, copy=True)
    idx = [int(i) for i in np.asarray(indices).reshape(-1)]
    B, T = np.asarray(q).shape[:2]
    segs = gdn_ref.segments(B, T, cu_seqlens)
    if len(idx) != len(segs):
        raise ValueError("one index per sequence")
    live = [n for n, s in enumerate(idx) if 0 <= s < pool.shape[0]]
    h0 = np.stack([pool[idx[n]] if n in live else np.zeros(pool.shape[1:], dtype)
                   for n in range(len(segs))])
    o, S = gdn_ref.recurrent(q, k, v, g, beta, scale=scale, initial_state=h0,
                             cu_seqlens=cu_seqlens, use_qk_l2norm=use_qk_l2norm, dtype=dtype)
    o = np.array(o, copy=True)
    for n, (b, s, e) in enumerate(segs):
        if n in live:
            pool[idx[n]] = S[n]
        else:
            o[b, s:e] = np.nan
    return o, pool
