"""Pinning checks for the backward oracle (oracle/gdn_bwd_ref.py), CPU only.

The reference repository has no gated delta rule, no backward and no
fixtures, so the backward oracle is pinned by what the mathematics fixes:

  finite differences  central differences of the fp64 forward definition
                      (oracle/gdn_ref.recurrent) for every input, with GQA,
                      an initial state, a final-state gradient, varlen with
                      an empty sequence, and the in-kernel l2norm
  library routine     torch.autograd through an independent torch
                      transcription of the forward (fp64)
  closed forms        beta = 0 (pure decay): dv = dk = 0, dq, dg, dh0 in
                      closed form
  identity            chunked backward == per-token backward for chunk
                      sizes 4, 16, 64 and ragged / packed sequences
  mutation checks     plausible mistakes planted in a copy of the per-token
                      backward (decay dropped from the state gradient, the
                      write's correction to dk dropped, dg read before the
                      decay) each fail the finite-difference check
"""
import numpy as np
import pytest
import torch

from oracle import gdn_bwd_ref as RB
from oracle import gdn_ref as R

RNG = np.random.default_rng


def _inputs(B=1, T=13, Hqk=2, Hv=4, K=5, V=3, seed=0, N=None, unit=True):
    rng = RNG(seed)
    q = rng.standard_normal((B, T, Hqk, K))
    k = rng.standard_normal((B, T, Hqk, K))
    if unit:
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, V))
    g = -0.3 * np.log1p(np.exp(rng.standard_normal((B, T, Hv))))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))
    N = B if N is None else N
    S0 = rng.standard_normal((N, Hv, K, V))
    do = rng.standard_normal((B, T, Hv, V))
    dht = rng.standard_normal((N, Hv, K, V))
    return dict(q=q, k=k, v=v, g=g, beta=beta, initial_state=S0), do, dht


def _loss(a, do, dht, **kw):
    o, S = R.recurrent(**a, **kw)
    return float((o * do).sum() + (S * dht).sum())


def _fd(a, do, dht, eps=1e-6, **kw):
    """Central finite differences of the loss for every input entry."""
    out = {}
    for name in ("q", "k", "v", "g", "beta", "initial_state"):
        x = a[name]
        fd = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            fd[i] = (_loss({**a, name: xp}, do, dht, **kw)
                     - _loss({**a, name: xm}, do, dht, **kw)) / (2 * eps)
        out[name] = fd
    return out


KEYS = dict(q="dq", k="dk", v="dv", g="dg", beta="dbeta", initial_state="dh0")


def _assert_fd(grads, fd, tol=1e-7):
    for name, key in KEYS.items():
        err = np.abs(grads[key] - fd[name]).max() / max(np.abs(fd[name]).max(), 1e-12)
        assert err < tol, f"{key}: relative error vs finite differences {err:.3e}"


@pytest.mark.parametrize("l2", [False, True])
def test_recurrent_bwd_matches_finite_differences(l2):
    a, do, dht = _inputs(seed=1)
    fd = _fd(a, do, dht, use_qk_l2norm=l2)
    gr = RB.recurrent_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                          initial_state=a["initial_state"], use_qk_l2norm=l2)
    _assert_fd(gr, fd)


def test_recurrent_bwd_varlen_matches_finite_differences():
    cu = np.array([0, 5, 5, 11])
    a, do, dht = _inputs(T=11, seed=2, N=3)
    fd = _fd(a, do, dht, cu_seqlens=cu)
    gr = RB.recurrent_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                          initial_state=a["initial_state"], cu_seqlens=cu)
    _assert_fd(gr, fd)


def _torch_forward(q, k, v, g, beta, S0, scale):
    """Independent torch transcription of the forward (V-major written as K-major)."""
    B, T, Hqk, K = q.shape
    Hv = v.shape[2]
    rep = Hv // Hqk
    qh = q.repeat_interleave(rep, dim=2)
    kh = k.repeat_interleave(rep, dim=2)
    S = S0[0]
    outs = []
    for t in range(T):
        S = S * torch.exp(g[0, t])[:, None, None]
        kv = torch.einsum("hkv,hk->hv", S, kh[0, t])
        delta = beta[0, t][:, None] * (v[0, t] - kv)
        S = S + kh[0, t][:, :, None] * delta[:, None, :]
        outs.append(scale * torch.einsum("hkv,hk->hv", S, qh[0, t]))
    return torch.stack(outs)[None], S[None]


def test_recurrent_bwd_matches_torch_autograd():
    a, do, dht = _inputs(T=40, Hqk=2, Hv=4, K=8, V=6, seed=3)
    ts = {n: torch.tensor(a[n], dtype=torch.float64, requires_grad=True)
          for n in ("q", "k", "v", "g", "beta", "initial_state")}
    o, S = _torch_forward(ts["q"], ts["k"], ts["v"], ts["g"], ts["beta"], ts["initial_state"],
                          8 ** -0.5)
    ((o * torch.tensor(do)).sum() + (S * torch.tensor(dht)).sum()).backward()
    gr = RB.recurrent_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                          initial_state=a["initial_state"])
    for name, key in KEYS.items():
        np.testing.assert_allclose(gr[key], ts[name].grad.numpy(), rtol=1e-10, atol=1e-12)


def test_pure_decay_closed_form():
    """beta = 0: S_t = e^{G_t} S0, o_t = c e^{G_t} S0^T q_t."""
    a, do, dht = _inputs(T=9, seed=4)
    a["beta"] = np.zeros_like(a["beta"])
    gr = RB.recurrent_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                          initial_state=a["initial_state"])
    c = a["q"].shape[-1] ** -0.5
    G = np.cumsum(a["g"][0], axis=0)                        # [T, Hv]
    S0 = a["initial_state"][0]
    hq = np.arange(4) // 2
    np.testing.assert_allclose(gr["dv"], 0, atol=0)
    np.testing.assert_allclose(gr["dk"], 0, atol=1e-15)
    # per-token contribution c e^{G_t} q^T S0 dO_t, and the final-state term
    contrib = c * np.exp(G) * np.einsum("thk,hkv,thv->th", a["q"][0][:, hq], S0, do[0])
    fin = np.exp(G[-1]) * (S0 * dht[0]).sum((1, 2))
    dg = np.cumsum(contrib[::-1], axis=0)[::-1] + fin[None, :]
    np.testing.assert_allclose(gr["dg"][0], dg, rtol=1e-12)
    dh0 = (c * np.einsum("th,thk,thv->hkv", np.exp(G), a["q"][0][:, hq], do[0])
           + np.exp(G[-1])[:, None, None] * dht[0])
    np.testing.assert_allclose(gr["dh0"][0], dh0, rtol=1e-12)
    dq = np.zeros_like(a["q"][0])
    for h in range(4):
        dq[:, hq[h]] += c * np.exp(G[:, h])[:, None] * (do[0][:, h] @ S0[h].T)
    np.testing.assert_allclose(gr["dq"][0], dq, rtol=1e-12)


@pytest.mark.parametrize("chunk", [4, 16, 64])
def test_chunked_bwd_equals_recurrent_bwd(chunk):
    a, do, dht = _inputs(T=70, Hqk=2, Hv=4, K=16, V=12, seed=5)
    gr = RB.recurrent_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                          initial_state=a["initial_state"])
    gc = RB.chunked_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                        initial_state=a["initial_state"], chunk=chunk)
    for key in gr:
        np.testing.assert_allclose(gc[key], gr[key], rtol=1e-9, atol=1e-10)


@pytest.mark.parametrize("l2", [False, True])
def test_chunked_bwd_varlen_equals_recurrent_bwd(l2):
    cu = np.array([0, 0, 21, 22, 57])
    a, do, dht = _inputs(T=57, Hqk=1, Hv=2, K=8, V=8, seed=6, N=4)
    gr = RB.recurrent_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                          initial_state=a["initial_state"], cu_seqlens=cu, use_qk_l2norm=l2)
    gc = RB.chunked_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                        initial_state=a["initial_state"], cu_seqlens=cu, use_qk_l2norm=l2,
                        chunk=16)
    for key in gr:
        np.testing.assert_allclose(gc[key], gr[key], rtol=1e-9, atol=1e-10)


def test_chunk_states_match_forward():
    a, _, _ = _inputs(T=50, K=8, V=8, seed=7)
    hs = RB.chunk_states(**a, chunk=16)[0]
    _, S = R.recurrent(**a)
    np.testing.assert_allclose(hs[-1], S[0], rtol=1e-12)
    _, S32 = R.recurrent(**{**a, "q": a["q"][:, :32], "k": a["k"][:, :32], "v": a["v"][:, :32],
                            "g": a["g"][:, :32], "beta": a["beta"][:, :32]})
    np.testing.assert_allclose(hs[2], S32[0], rtol=1e-12)


# ----------------------------------------------------------- mutation checks --

def _mutant_bwd(a, do, dht, bug):
    """Per-token backward written out once more, with one planted mistake."""
    q, k, v, g, beta, S0 = (a[n] for n in ("q", "k", "v", "g", "beta", "initial_state"))
    B, T, Hqk, K = q.shape
    Hv = v.shape[2]
    hq = np.arange(Hv) // (Hv // Hqk)
    c = K ** -0.5
    S = S0[0].copy()
    Sp = []
    for t in range(T):
        Sp.append(S)
        S = np.exp(g[0, t])[:, None, None] * S
        u = np.einsum("hkv,hk->hv", S, k[0, t, hq])
        S = S + k[0, t, hq][:, :, None] * (beta[0, t][:, None] * (v[0, t] - u))[:, None, :]
    out = {key: np.zeros_like(a[n]) for n, key in KEYS.items()}
    D = dht[0].copy()
    for t in range(T - 1, -1, -1):
        kt, qt, eg = k[0, t, hq], q[0, t, hq], np.exp(g[0, t])
        Sb = eg[:, None, None] * Sp[t]
        u = np.einsum("hkv,hk->hv", Sb, kt)
        d = beta[0, t][:, None] * (v[0, t] - u)
        St = Sb + kt[:, :, None] * d[:, None, :]
        D = D + c * qt[:, :, None] * do[0, t][:, None, :]
        np.add.at(out["dq"][0, t], hq, c * np.einsum("hkv,hv->hk", St, do[0, t]))
        dd = np.einsum("hkv,hk->hv", D, kt)
        out["dv"][0, t] = beta[0, t][:, None] * dd
        out["dbeta"][0, t] = ((v[0, t] - u) * dd).sum(-1)
        du = -beta[0, t][:, None] * dd
        dk = np.einsum("hkv,hv->hk", D, d)
        if bug != "no_read_term":
            dk = dk + np.einsum("hkv,hv->hk", Sb, du)
        np.add.at(out["dk"][0, t], hq, dk)
        E = D + kt[:, :, None] * du[:, None, :]
        out["dg"][0, t] = ((Sp[t] if bug == "dg_before_decay" else Sb) * E).sum((1, 2))
        D = E if bug == "no_decay" else eg[:, None, None] * E
    out["dh0"][0] = D
    return out


@pytest.mark.parametrize("bug", ["no_decay", "no_read_term", "dg_before_decay"])
def test_planted_mistakes_fail_finite_differences(bug):
    a, do, dht = _inputs(T=7, Hqk=1, Hv=2, K=4, V=3, seed=8)
    fd = _fd(a, do, dht)
    _assert_fd(_mutant_bwd(a, do, dht, None), fd)       # the unmutated copy passes
    with pytest.raises(AssertionError):
        _assert_fd(_mutant_bwd(a, do, dht, bug), fd)
