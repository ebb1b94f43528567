"""numpy oracle for the gated delta rule BACKWARD (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import this
module; the product never does.

Forward (per sequence and v-head, K-major state S [K, V], c = scale):

    Sb_t = e^{g_t} S_{t-1};  u_t = Sb_t^T k_t;  d_t = beta_t (v_t - u_t)
    S_t  = Sb_t + k_t d_t^T;  o_t = c S_t^T q_t

Given dO and dS_T (gradient of the returned final state), ``recurrent_bwd``
runs the definition backwards token by token (D_t = dL/dS_t):

    D_t   += c q_t dO_t^T                   (o_t reads S_t)
    dq_t   = c S_t dO_t
    dd     = D_t^T k_t;  dv_t = beta_t dd;  dbeta_t = (v_t - u_t) . dd
    du     = -beta_t dd
    dk_t   = D_t d_t + Sb_t du
    E_t    = D_t + k_t du^T                 (dL/dSb_t)
    dg_t   = <Sb_t, E_t>
    D_t-1  = e^{g_t} E_t                    (D before the sequence = dh0)

``chunked_bwd`` is the chunk-level restatement the GPU kernels follow
(reverse-mode differentiation of the chunked forward of gdn_ref.chunked,
chunk C): the forward chain gives each chunk's start state S_c; a reverse
chain gives dS'_c, the gradient flowing into the chunk's end state,

    dd    = P~^T dO' + Kt dS'               dO' = c dO, Kt_j = e^{G_L - G_j} k_j
    dS_c  = e^{G_L} dS' + (e^G * Q)^T dO' - (e^G * K)^T (Tb^T dd)

with P~ = lower_incl(Q K^T * Gam), Tb = (I + A)^-1 diag(beta); each chunk's
gradients are then local (``_chunk_grads``).  Both functions also accept
``use_qk_l2norm`` (chain rule through x / sqrt(|x|^2 + 1e-6)) and sum dq, dk
over the v-heads of a qk-head group.

The reference repository (848267592/avelang) has no gated delta rule, so
there is nothing to follow there; the forward's conventions are those of
transformers' modeling_qwen3_next.py:368-503 (read as text).  The backward
is derived from the forward above.  Pinning (tests/test_oracle_bwd.py):
central finite differences of gdn_ref.recurrent in fp64, torch.autograd
through an independent torch transcription of the forward, closed forms
and the chunked == recurrent identity.
"""
from __future__ import annotations

import numpy as np

from . import gdn_ref as R

__all__ = ["recurrent_bwd", "chunked_bwd", "l2norm_bwd", "chunk_states"]


def l2norm_bwd(x, dy, eps: float = 1e-6):
    """Gradient of y = x / sqrt(sum(x^2) + eps) over the last axis."""
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) + eps)
    y = x * r
    return r * (dy - y * (y * dy).sum(-1, keepdims=True))


def _setup(q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype):
    q0 = np.asarray(q, dtype=dtype)
    k0 = np.asarray(k, dtype=dtype)
    q, k, v, g, beta, scale, S0, segs, hq = R._prep(
        q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype)
    return q0, k0, q, k, v, g, beta, scale, S0, segs, hq


def _finish(dq, dk, q0, k0, use_qk_l2norm):
    if use_qk_l2norm:
        dq = l2norm_bwd(q0, dq)
        dk = l2norm_bwd(k0, dk)
    return dq, dk


def recurrent_bwd(q, k, v, g, beta, do, dht=None, scale=None, initial_state=None,
                  cu_seqlens=None, use_qk_l2norm=False, dtype=np.float64):
    """Token-by-token backward of the recurrence (the definition).

    Returns dict(dq, dk [B,T,Hqk,K], dv [B,T,Hv,V], dg, dbeta [B,T,Hv],
    dh0 [N,Hv,K,V]).  ``dht`` is the gradient of the final state (None = 0).
    """
    q0, k0, q, k, v, g, beta, scale, S0, segs, hq = _setup(
        q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype)
    do = np.asarray(do, dtype=dtype)
    B, T, Hqk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    dq = np.zeros((B, T, Hqk, K), dtype)
    dk = np.zeros((B, T, Hqk, K), dtype)
    dv = np.zeros((B, T, Hv, V), dtype)
    dg = np.zeros((B, T, Hv), dtype)
    db = np.zeros((B, T, Hv), dtype)
    dh0 = np.zeros((len(segs), Hv, K, V), dtype)
    for n, (b, s, e) in enumerate(segs):
        # forward, keeping the state before every token
        S = S0[n].copy()
        Sprev = np.zeros((e - s, Hv, K, V), dtype)
        for t in range(s, e):
            Sprev[t - s] = S
            S = np.exp(g[b, t])[:, None, None] * S
            u = np.einsum("hkv,hk->hv", S, k[b, t, hq])
            S = S + k[b, t, hq][:, :, None] * (beta[b, t][:, None] * (v[b, t] - u))[:, None, :]
        D = np.zeros((Hv, K, V), dtype) if dht is None else np.array(dht[n], dtype=dtype)
        for t in range(e - 1, s - 1, -1):
            qt, kt = q[b, t, hq], k[b, t, hq]
            eg = np.exp(g[b, t])
            Sb = eg[:, None, None] * Sprev[t - s]
            u = np.einsum("hkv,hk->hv", Sb, kt)
            d = beta[b, t][:, None] * (v[b, t] - u)
            St = Sb + kt[:, :, None] * d[:, None, :]
            D = D + scale * qt[:, :, None] * do[b, t][:, None, :]
            np.add.at(dq[b, t], hq, scale * np.einsum("hkv,hv->hk", St, do[b, t]))
            dd = np.einsum("hkv,hk->hv", D, kt)
            dv[b, t] = beta[b, t][:, None] * dd
            db[b, t] = ((v[b, t] - u) * dd).sum(-1)
            du = -beta[b, t][:, None] * dd
            np.add.at(dk[b, t], hq, np.einsum("hkv,hv->hk", D, d) + np.einsum("hkv,hv->hk", Sb, du))
            E = D + kt[:, :, None] * du[:, None, :]
            dg[b, t] = (Sb * E).sum((1, 2))
            D = eg[:, None, None] * E
        dh0[n] = D
    dq, dk = _finish(dq, dk, q0, k0, use_qk_l2norm)
    return dict(dq=dq, dk=dk, dv=dv, dg=dg, dbeta=db, dh0=dh0)


# ------------------------------------------------------------- chunked form --

def _chunk_fwd_parts(Qc, Kc, Vc, gc, bc, dtype):
    """Per-chunk quantities of the forward (all heads at once).

    Qc, Kc [Hv, L, K]; Vc [Hv, L, V]; gc, bc [Hv, L].  Returns a dict with
    G, Gam (masked to i >= j), T = (I + A)^-1, A, KK = K K^T, QK = Q K^T.
    """
    L = Qc.shape[1]
    G = np.cumsum(gc, axis=1, dtype=dtype)
    low = np.tril(np.ones((L, L), dtype=bool))
    Gam = np.where(low, np.exp(np.where(low, G[:, :, None] - G[:, None, :], 0.0)), 0.0).astype(dtype)
    KK = Kc @ Kc.transpose(0, 2, 1)
    QK = Qc @ Kc.transpose(0, 2, 1)
    A = np.tril(bc[:, :, None] * KK * Gam, -1)
    Tm = R.ut_inverse(A)
    return dict(G=G, Gam=Gam, KK=KK, QK=QK, A=A, T=Tm)


def chunk_states(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None,
                 use_qk_l2norm=False, chunk=64, dtype=np.float64):
    """Forward chain only: the state at the start of every chunk.

    Returns (list over sequences of [nchunks + 1, Hv, K, V] arrays, the last
    entry being the final state) -- what the GPU forward-with-save stores.
    """
    _, _, q, k, v, g, beta, scale, S0, segs, hq = _setup(
        q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype)
    out = []
    for n, (b, s, e) in enumerate(segs):
        S = S0[n].copy()
        hs = [S.copy()]
        for a in range(s, e, chunk):
            z = min(a + chunk, e)
            Qc = q[b, a:z][:, hq].transpose(1, 0, 2)
            Kc = k[b, a:z][:, hq].transpose(1, 0, 2)
            Vc = v[b, a:z].transpose(1, 0, 2)
            gc, bc = g[b, a:z].T, beta[b, a:z].T
            f = _chunk_fwd_parts(Qc, Kc, Vc, gc, bc, dtype)
            eG = np.exp(f["G"])
            d = f["T"] @ (bc[:, :, None] * (Vc - eG[:, :, None] * (Kc @ S)))
            dec = np.exp(f["G"][:, -1:] - f["G"])
            S = np.exp(f["G"][:, -1])[:, None, None] * S + (Kc * dec[:, :, None]).transpose(0, 2, 1) @ d
            hs.append(S.copy())
        out.append(np.stack(hs))
    return out


def _chunk_grads(Qc, Kc, Vc, gc, bc, S, dSe, dOc, scale, dtype):
    """Local gradients of one chunk (all v-heads at once).

    S = the chunk's start state, dSe = dL/d(end state) from later chunks,
    dOc = dL/do of the chunk's rows.  Returns (dQ, dK, dV, dg, dbeta, dS)
    with dS = dL/dS (to the previous chunk).  Every line is one step of
    reverse-mode differentiation of the chunk forward:

        Tb = T diag(b);  d = Tb (V - e^G * (K S))      (= u - w S)
        O  = c [e^G * (Q S) + P~ d],  P~ = lower_incl(Q K^T * Gam)
        S' = e^{G_L} S + Kt^T d,  Kt = e^{G_L - G} * K
    """
    f = _chunk_fwd_parts(Qc, Kc, Vc, gc, bc, dtype)
    G, Gam, KK, QK, Tm = f["G"], f["Gam"], f["KK"], f["QK"], f["T"]
    L = Qc.shape[1]
    eG = np.exp(G)                                   # [H, L]
    GL = G[:, -1]
    eGL = np.exp(GL)
    dec = np.exp(GL[:, None] - G)                    # e^{G_L - G_j}
    KS = Kc @ S                                      # [H, L, V]
    d = Tm @ (bc[:, :, None] * (Vc - eG[:, :, None] * KS))
    Pt = np.tril(QK * Gam)                           # incl. diagonal (Gam_ii = 1)
    Kt = Kc * dec[:, :, None]
    dO = scale * dOc                                 # dO'
    # reverse chain terms
    dd = Pt.transpose(0, 2, 1) @ dO + Kt @ dSe       # dL/dd
    dS = (eGL[:, None, None] * dSe + (Qc * eG[:, :, None]).transpose(0, 2, 1) @ dO)
    # O = c e^G (Q S) + ...:
    dQ = eG[:, :, None] * (dO @ S.transpose(0, 2, 1))
    dGv = eG * np.einsum("hlk,hlk->hl", Qc, dO @ S.transpose(0, 2, 1))   # d/dG_i via e^{G_i}
    dPt = np.tril(dO @ d.transpose(0, 2, 1))
    # S' = e^{G_L} S + Kt^T d
    dGL = eGL * (S * dSe).sum((1, 2))
    dKt = d @ dSe.transpose(0, 2, 1)                 # [H, L, K]
    dK = dec[:, :, None] * dKt
    rho = (Kt * dKt).sum(-1)                         # d/d(G_L - G_j)
    dGL = dGL + rho.sum(-1)
    dGv = dGv - rho
    # d = u - w S with u = T diag(b) V, w = T diag(b e^G) K
    dU = dd
    dW = -(dd @ S.transpose(0, 2, 1))                # [H, L, K]
    TtdU = Tm.transpose(0, 2, 1) @ dU                # T^T dU
    dS = dS - ((bc * eG)[:, :, None] * Kc).transpose(0, 2, 1) @ TtdU   # - w^T dd
    TtdW = Tm.transpose(0, 2, 1) @ dW
    dV = bc[:, :, None] * TtdU
    dbv = (Vc * TtdU).sum(-1) + eG * (Kc * TtdW).sum(-1)
    dK = dK + (bc * eG)[:, :, None] * TtdW
    dGv = dGv + bc * eG * (Kc * TtdW).sum(-1)
    Vb = bc[:, :, None] * Vc
    Kb = (bc * eG)[:, :, None] * Kc
    dT = dU @ Vb.transpose(0, 2, 1) + dW @ Kb.transpose(0, 2, 1)
    dA = -(Tm.transpose(0, 2, 1) @ dT @ Tm.transpose(0, 2, 1))
    dA = np.tril(dA, -1)
    # A_ij = b_i KK_ij Gam_ij (i > j)
    dbv = dbv + (dA * KK * Gam).sum(-1)
    M = dA * bc[:, :, None] * Gam
    dK = dK + M @ Kc + M.transpose(0, 2, 1) @ Kc
    dGam = dA * bc[:, :, None] * KK
    # P~_ij = QK_ij Gam_ij (i >= j)
    MP = dPt * Gam
    dQ = dQ + MP @ Kc
    dK = dK + MP.transpose(0, 2, 1) @ Qc
    dGam = dGam + dPt * QK
    # Gam_ij = e^{G_i - G_j}
    X = dGam * Gam
    dGv = dGv + X.sum(-1) - X.sum(-2)
    dGv[:, L - 1] += dGL
    # G = cumsum(g): dg_i = sum_{m >= i} dG_m
    dg = np.cumsum(dGv[:, ::-1], axis=1)[:, ::-1]
    return dQ, dK, dV, dg, dbv, dS


def chunked_bwd(q, k, v, g, beta, do, dht=None, scale=None, initial_state=None,
                cu_seqlens=None, use_qk_l2norm=False, chunk=64, dtype=np.float64):
    """Chunk-level backward (what the GPU path computes); same returns as recurrent_bwd."""
    q0, k0, q, k, v, g, beta, scale, S0, segs, hq = _setup(
        q, k, v, g, beta, scale, initial_state, cu_seqlens, use_qk_l2norm, dtype)
    do = np.asarray(do, dtype=dtype)
    B, T, Hqk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    G_ = Hv // Hqk
    hs_all = chunk_states(q, k, v, g, beta, scale, S0, cu_seqlens, False, chunk, dtype)
    dq = np.zeros((B, T, Hqk, K), dtype)
    dk = np.zeros((B, T, Hqk, K), dtype)
    dv = np.zeros((B, T, Hv, V), dtype)
    dg = np.zeros((B, T, Hv), dtype)
    db = np.zeros((B, T, Hv), dtype)
    dh0 = np.zeros((len(segs), Hv, K, V), dtype)
    for n, (b, s, e) in enumerate(segs):
        hs = hs_all[n]
        dSe = np.zeros((Hv, K, V), dtype) if dht is None else np.array(dht[n], dtype=dtype)
        starts = list(range(s, e, chunk))
        for c in range(len(starts) - 1, -1, -1):
            a = starts[c]
            z = min(a + chunk, e)
            Qc = q[b, a:z][:, hq].transpose(1, 0, 2)
            Kc = k[b, a:z][:, hq].transpose(1, 0, 2)
            Vc = v[b, a:z].transpose(1, 0, 2)
            gc, bc = g[b, a:z].T, beta[b, a:z].T
            dOc = do[b, a:z].transpose(1, 0, 2)
            dQ, dK, dV, dgc, dbc, dSe = _chunk_grads(Qc, Kc, Vc, gc, bc, hs[c], dSe, dOc,
                                                      scale, dtype)
            # sum over the v-heads of each qk-head group
            dq[b, a:z] += dQ.reshape(Hqk, G_, z - a, K).sum(1).transpose(1, 0, 2)
            dk[b, a:z] += dK.reshape(Hqk, G_, z - a, K).sum(1).transpose(1, 0, 2)
            dv[b, a:z] = dV.transpose(1, 0, 2)
            dg[b, a:z] = dgc.T
            db[b, a:z] = dbc.T
        dh0[n] = dSe
    dq, dk = _finish(dq, dk, q0, k0, use_qk_l2norm)
    return dict(dq=dq, dk=dk, dv=dv, dg=dg, dbeta=db, dh0=dh0)
