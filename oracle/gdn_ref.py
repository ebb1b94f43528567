"""numpy oracle for the gated delta rule (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product never does.

Semantics (per v-head h, qk-head ``h // (Hv // Hqk)``; state S is [K, V]):

    S  <- exp(g_t) * S
    kv  = S^T k_t                      (reduce over K)
    d   = beta_t * (v_t - kv)
    S  <- S + k_t (outer) d
    o_t = scale * S^T q_t

Layouts: q, k [B, T, Hqk, K]; v, o [B, T, Hv, V]; g, beta [B, T, Hv];
state [N, Hv, K, V].  With ``cu_seqlens`` B must be 1 and N = len - 1.

The reference repository contains no gated delta rule; the conventions
(default scale K**-0.5, l2norm eps 1e-6, zero padding of the tail chunk,
output read after the update) follow
transformers/models/qwen3_next/modeling_qwen3_next.py:368-503 (third
party, read as text).  Pinning checks live in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "l2norm",
    "segments",
    "recurrent",
    "ut_inverse",
    "chunked",
]


def l2norm(x, eps: float = 1e-6):
    """x * rsqrt(sum(x^2) + eps) over the last axis (modeling_qwen3_next.py:368-371)."""
    x = np.asarray(x)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def segments(B: int, T: int, cu_seqlens=None):
    """List of (batch, start, end) sequences.

    Without cu_seqlens every batch row is one sequence of length T; with
    cu_seqlens (B must be 1) sequence n covers tokens [cu[n], cu[n+1]).
    """
    if cu_seqlens is None:
        return [(b, 0, T) for b in range(B)]
    cu = [int(c) for c in np.asarray(cu_seqlens).reshape(-1)]
    if B != 1:
        raise ValueError("cu_seqlens requires B == 1")
    if cu[0] != 0 or cu[-1] != T or any(b < a for a, b in zip(cu[:-1], cu[1:])):
        raise ValueError("cu_seqlens must be non-decreasing from 0 to T")
    return [(0, a, b) for a, b in zip(cu[:-1], cu[1:])]


def _prep(q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype):
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    g = np.asarray(g, dtype=dtype)
    beta = np.asarray(beta, dtype=dtype)
    B, T, Hqk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    if k.shape != q.shape or v.shape[:2] != (B, T) or g.shape != (B, T, Hv) or beta.shape != (B, T, Hv):
        raise ValueError("inconsistent shapes")
    if Hv % Hqk:
        raise ValueError("Hv must be a multiple of Hqk")
    if use_qk_l2norm:
        q = l2norm(q).astype(dtype)
        k = l2norm(k).astype(dtype)
    if scale is None:
        scale = K ** -0.5
    segs = segments(B, T, cu_seqlens)
    N = len(segs)
    if initial_state is None:
        S0 = np.zeros((N, Hv, K, V), dtype=dtype)
    else:
        S0 = np.array(initial_state, dtype=dtype, copy=True)
        if S0.shape != (N, Hv, K, V):
            raise ValueError(f"initial_state must be {(N, Hv, K, V)}")
    hq = np.arange(Hv) // (Hv // Hqk)
    return q, k, v, g, beta, dtype(scale) if callable(dtype) else scale, S0, segs, hq


def recurrent(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None,
              use_qk_l2norm=False, dtype=np.float64):
    """Per-token gated delta rule: the definition.

    Follows the token loop of torch_recurrent_gated_delta_rule
    (modeling_qwen3_next.py:490-501).  Returns (o [B,T,Hv,V], S [N,Hv,K,V]).
    """
    q, k, v, g, beta, scale, S_all, segs, hq = _prep(
        q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype)
    B, T = q.shape[:2]
    Hv, V = v.shape[2], v.shape[3]
    o = np.zeros((B, T, Hv, V), dtype=dtype)
    for n, (b, s, e) in enumerate(segs):
        S = S_all[n]
        for t in range(s, e):
            qt = q[b, t, hq]                      # [Hv, K]
            kt = k[b, t, hq]
            S *= np.exp(g[b, t])[:, None, None]
            kv = np.einsum("hkv,hk->hv", S, kt)
            d = beta[b, t][:, None] * (v[b, t] - kv)
            S += kt[:, :, None] * d[:, None, :]
            o[b, t] = scale * np.einsum("hkv,hk->hv", S, qt)
    return o, S_all


def ut_inverse(A):
    """(I + A)^-1 for strictly lower-triangular A [..., L, L] by forward substitution.

    Row form of the in-place loop at modeling_qwen3_next.py:420-424
    (which builds -(I+A)^-1 + 2I from -A); here the inverse itself.
    """
    A = np.asarray(A)
    L = A.shape[-1]
    Tm = np.zeros_like(A)
    eye = np.eye(L, dtype=A.dtype)
    for i in range(L):
        Tm[..., i, :] = eye[i] - np.einsum("...j,...jc->...c", A[..., i, :i], Tm[..., :i, :])
    return Tm


def chunked(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None,
            use_qk_l2norm=False, chunk=64, dtype=np.float32):
    """Chunked (UT/WY) form of the same recurrence, in ``dtype`` (fp32).

    Per chunk of <= ``chunk`` tokens of one sequence (chunks never straddle
    sequences; a short tail chunk equals zero padding,
    modeling_qwen3_next.py:397-403):

        Gc   = cumsum(g)                                   (:417)
        Gam  = exp(Gc_i - Gc_j), i >= j                    (:418)
        A    = strict_lower(diag(beta) K K^T * Gam)        (:419)
        Tm   = (I + A)^-1                                  (:420-424)
        u    = Tm diag(beta) V ; w = Tm diag(beta e^Gc) K  (:425-426)
        vnew = u - w S                                     (:439-440)
        o    = scale [e^Gc * (Q S) + tril(Q K^T * Gam) vnew]  (:438, 441-442)
        S    = e^Gc_L S + (K * e^(Gc_L - Gc))^T vnew       (:443-446)
    """
    q, k, v, g, beta, scale, S_all, segs, hq = _prep(
        q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype)
    B, T = q.shape[:2]
    Hv, V = v.shape[2], v.shape[3]
    o = np.zeros((B, T, Hv, V), dtype=dtype)
    for n, (b, s, e) in enumerate(segs):
        S = S_all[n]
        for a in range(s, e, chunk):
            z = min(a + chunk, e)
            L = z - a
            Qc = q[b, a:z][:, hq].transpose(1, 0, 2)      # [Hv, L, K]
            Kc = k[b, a:z][:, hq].transpose(1, 0, 2)
            Vc = v[b, a:z].transpose(1, 0, 2)             # [Hv, L, V]
            gc = g[b, a:z].T                              # [Hv, L]
            bc = beta[b, a:z].T
            Gc = np.cumsum(gc, axis=1, dtype=dtype)
            low = np.tril(np.ones((L, L), dtype=bool))
            diff = np.where(low, Gc[:, :, None] - Gc[:, None, :], -np.inf)
            Gam = np.exp(diff).astype(dtype)
            A = bc[:, :, None] * (Kc @ Kc.transpose(0, 2, 1)) * Gam
            A = np.tril(A, -1)
            Tm = ut_inverse(A)
            eG = np.exp(Gc)
            u = Tm @ (bc[:, :, None] * Vc)
            w = Tm @ ((bc * eG)[:, :, None] * Kc)
            vnew = u - w @ S
            P = (Qc @ Kc.transpose(0, 2, 1)) * Gam
            oc = scale * (eG[:, :, None] * (Qc @ S) + P @ vnew)
            o[b, a:z] = oc.transpose(1, 0, 2)
            dec = np.exp(Gc[:, -1:] - Gc)                 # [Hv, L]
            S *= np.exp(Gc[:, -1])[:, None, None]
            S += (Kc * dec[:, :, None]).transpose(0, 2, 1) @ vnew
    return o, S_all
