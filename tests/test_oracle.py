"""Pinning checks for the CPU oracle (runs without a GPU).

The reference repository ships no gated-delta-rule code, tests or fixtures,
so the oracle (oracle/gdn_ref.py, oracle/gdn_cpu.c) is pinned by what the
mathematics fixes, each check written independently of the oracle's code:

  closed forms      beta = 0 (pure decay), g = beta = 0 (constant state),
                    S0 = 0 and T = 1 (one outer product), exact retrieval
                    for unit k with beta = 1, g = 0
  invariants        per-step retrieval identity for unit k, joint linearity
                    in (S0, v), split-resume, varlen == independent runs,
                    GQA == explicit head repetition
  textbook routine  UT inverse vs scipy.linalg.solve_triangular
  brute force       fp64 recurrence vs fp32 chunked form vs the C port
  mutation checks   plausible mistakes planted in copies of the recurrence
                    (transposed state, decay after the read, beta dropped
                    from the write, wrong GQA map) each fail a check above
"""
import numpy as np
import pytest
import scipy.linalg

from oracle import cpu as coracle
from oracle import gdn_ref as R

RNG = np.random.default_rng


def _inputs(B=1, T=50, Hqk=2, Hv=4, K=16, V=24, seed=0, h0=True, unit=True, N=None):
    rng = RNG(seed)
    q = rng.standard_normal((B, T, Hqk, K))
    k = rng.standard_normal((B, T, Hqk, K))
    if unit:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, V))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))
    g = -0.1 * np.log1p(np.exp(rng.standard_normal((B, T, Hv))))
    N = B if N is None else N
    S0 = 0.1 * rng.standard_normal((N, Hv, K, V)) if h0 else None
    return dict(q=q, k=k, v=v, g=g, beta=beta, initial_state=S0)


def _gqa(h, Hqk, Hv):
    return h // (Hv // Hqk)


# ---------------------------------------------------------------- closed forms

def test_pure_decay_when_beta_zero():
    a = _inputs(seed=1)
    a["beta"] = np.zeros_like(a["beta"])
    o, S = R.recurrent(**a)
    scale = a["q"].shape[-1] ** -0.5
    G = np.cumsum(a["g"][0], axis=0)                       # [T, Hv]
    S0 = a["initial_state"][0]
    for h in range(4):
        hq = _gqa(h, 2, 4)
        for t in (0, 17, 49):
            want = scale * np.exp(G[t, h]) * np.array(
                [sum(S0[h, i, j] * a["q"][0, t, hq, i] for i in range(16)) for j in range(24)])
            np.testing.assert_allclose(o[0, t, h], want, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(S[0, h], np.exp(G[-1, h]) * S0[h], rtol=1e-12)


def test_constant_state_when_g_and_beta_zero():
    a = _inputs(seed=2)
    a["beta"] = np.zeros_like(a["beta"])
    a["g"] = np.zeros_like(a["g"])
    o, S = R.recurrent(**a)
    np.testing.assert_allclose(S, a["initial_state"], rtol=0, atol=0)


def test_single_token_from_zero_state_is_outer_product():
    """S1[i, j] = beta k_i v_j (K-major orientation) and o = scale beta (q.k) v."""
    a = _inputs(T=1, seed=3, h0=False)
    o, S = R.recurrent(**a)
    scale = 16 ** -0.5
    for h in range(4):
        hq = _gqa(h, 2, 4)
        kk, vv, qq, bb = a["k"][0, 0, hq], a["v"][0, 0, h], a["q"][0, 0, hq], a["beta"][0, 0, h]
        want = np.empty((16, 24))
        for i in range(16):
            for j in range(24):
                want[i, j] = bb * kk[i] * vv[j]
        np.testing.assert_allclose(S[0, h], want, rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(o[0, 0, h], scale * bb * float(qq @ kk) * vv, rtol=1e-12)


def test_exact_retrieval_unit_key_beta_one():
    a = _inputs(T=7, seed=4)
    a["beta"] = np.ones_like(a["beta"])
    a["g"] = np.zeros_like(a["g"])
    _, S = R.recurrent(**a)
    for h in range(4):
        kT = a["k"][0, -1, _gqa(h, 2, 4)]
        np.testing.assert_allclose(kT @ S[0, h], a["v"][0, -1, h], rtol=1e-10, atol=1e-12)


def test_per_step_retrieval_identity():
    """unit k: S_t^T k_t = (1 - beta_t) e^g_t S_{t-1}^T k_t + beta_t v_t."""
    a = _inputs(T=30, seed=5)
    for t in (1, 12, 29):
        prev = {kk: (x[:, :t] if x is not None and kk != "initial_state" else x) for kk, x in a.items()}
        cur = {kk: (x[:, :t + 1] if x is not None and kk != "initial_state" else x) for kk, x in a.items()}
        _, Sp = R.recurrent(**prev)
        _, Sc = R.recurrent(**cur)
        for h in range(4):
            kt = a["k"][0, t, _gqa(h, 2, 4)]
            b, g = a["beta"][0, t, h], a["g"][0, t, h]
            want = (1 - b) * np.exp(g) * (kt @ Sp[0, h]) + b * a["v"][0, t, h]
            np.testing.assert_allclose(kt @ Sc[0, h], want, rtol=1e-10, atol=1e-12)


# ------------------------------------------------------------------ invariants

def test_joint_linearity_in_state_and_values():
    a = _inputs(seed=6)
    b = dict(a)
    rng = RNG(60)
    b["v"] = rng.standard_normal(a["v"].shape)
    b["initial_state"] = rng.standard_normal(a["initial_state"].shape)
    c = dict(a)
    c["v"] = 2.0 * a["v"] - 3.0 * b["v"]
    c["initial_state"] = 2.0 * a["initial_state"] - 3.0 * b["initial_state"]
    oa, Sa = R.recurrent(**a)
    ob, Sb = R.recurrent(**b)
    oc, Sc = R.recurrent(**c)
    np.testing.assert_allclose(oc, 2 * oa - 3 * ob, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(Sc, 2 * Sa - 3 * Sb, rtol=1e-9, atol=1e-11)


def test_split_resume():
    a = _inputs(T=90, seed=7)
    o, S = R.recurrent(**a)
    first = {kk: (x[:, :37] if kk != "initial_state" else x) for kk, x in a.items()}
    o1, S1 = R.recurrent(**first)
    second = {kk: x[:, 37:] for kk, x in a.items() if kk != "initial_state"}
    o2, S2 = R.recurrent(**second, initial_state=S1)
    np.testing.assert_allclose(np.concatenate([o1, o2], 1), o, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(S2, S, rtol=1e-12, atol=1e-14)


def test_varlen_equals_independent_sequences():
    cu = np.array([0, 11, 11, 40, 64])
    a = _inputs(T=64, seed=8, N=4)
    o, S = R.recurrent(**a, cu_seqlens=cu)
    for n in range(4):
        lo, hi = cu[n], cu[n + 1]
        part = {kk: x[:, lo:hi] for kk, x in a.items() if kk != "initial_state"}
        on, Sn = R.recurrent(**part, initial_state=a["initial_state"][n:n + 1])
        np.testing.assert_allclose(o[:, lo:hi], on, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(S[n], Sn[0], rtol=1e-12, atol=1e-14)


def test_gqa_equals_explicit_head_repetition():
    a = _inputs(seed=9, Hqk=2, Hv=4)
    o, S = R.recurrent(**a)
    rep = dict(a)
    rep["q"] = np.repeat(a["q"], 2, axis=2)
    rep["k"] = np.repeat(a["k"], 2, axis=2)
    o2, S2 = R.recurrent(**rep)
    np.testing.assert_allclose(o, o2, rtol=0, atol=0)
    np.testing.assert_allclose(S, S2, rtol=0, atol=0)
    # the map must not be the identity or a modulo: heads 0, 1 share qk-head 0
    assert not np.allclose(o[..., 0, :], R.recurrent(**dict(a, q=a["q"][:, :, ::-1], k=a["k"][:, :, ::-1]))[0][..., 0, :])


def test_l2norm_option_matches_prenormalised_inputs():
    a = _inputs(seed=10, unit=False)
    o, S = R.recurrent(**a, use_qk_l2norm=True)
    b = dict(a)
    b["q"] = a["q"] / np.sqrt((a["q"] ** 2).sum(-1, keepdims=True) + 1e-6)
    b["k"] = a["k"] / np.sqrt((a["k"] ** 2).sum(-1, keepdims=True) + 1e-6)
    o2, S2 = R.recurrent(**b)
    np.testing.assert_allclose(o, o2, rtol=1e-12)
    np.testing.assert_allclose(S, S2, rtol=1e-12)


def test_l2norm_eps_inside_the_square_root():
    """R.l2norm against what the formula x / sqrt(|x|^2 + eps), eps = 1e-6, fixes at both
    ends, with the norm from numpy.linalg.norm: a large-norm row comes out unit-norm, and a
    row of norm 1e-5 (|x|^2 = 1e-10, negligible beside eps) is scaled by eps^-1/2 = 1000.
    Planted mistakes fail: eps outside the square root (x / (|x| + eps) scales the tiny
    row by ~9e4), eps dropped (unit norm for the tiny row), eps squared inside."""
    rng = np.random.default_rng(31)
    big = rng.standard_normal((3, 128)) * 7.0
    tiny = rng.standard_normal((3, 128))
    tiny *= 1e-5 / np.linalg.norm(tiny, axis=-1, keepdims=True)
    nb = R.l2norm(big)
    np.testing.assert_allclose(np.linalg.norm(nb, axis=-1), 1.0, rtol=1e-7)
    np.testing.assert_allclose(nb, big / np.linalg.norm(big, axis=-1, keepdims=True), rtol=1e-7)
    nt = R.l2norm(tiny)
    np.testing.assert_allclose(nt, tiny * 1e3, rtol=1e-4)
    np.testing.assert_allclose(np.linalg.norm(nt, axis=-1), 1e-2, rtol=1e-4)
    mistakes = [lambda x: x / (np.linalg.norm(x, axis=-1, keepdims=True) + 1e-6),
                lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True),
                lambda x: x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-12)]
    for bad in mistakes:
        assert not np.allclose(bad(tiny), nt, rtol=1e-2)


def test_default_scale_is_inverse_sqrt_k():
    a = _inputs(seed=11)
    o, _ = R.recurrent(**a)
    o2, _ = R.recurrent(**a, scale=0.25)            # K = 16 -> 1/4
    np.testing.assert_array_equal(o, o2)


# ------------------------------------------------------------ textbook routine

@pytest.mark.parametrize("L", [1, 5, 16, 64])
def test_ut_inverse_matches_solve_triangular(L):
    rng = RNG(L)
    A = np.tril(rng.standard_normal((3, L, L)) * 0.3, -1)
    Tm = R.ut_inverse(A)
    eye = np.eye(L)
    for i in range(3):
        ref = scipy.linalg.solve_triangular(eye + A[i], eye, lower=True, unit_diagonal=True)
        np.testing.assert_allclose(Tm[i], ref, rtol=1e-10, atol=1e-12)
        assert np.abs((eye + A[i]) @ Tm[i] - eye).max() <= 1e-10


# ----------------------------------------------------------------- brute force

@pytest.mark.parametrize("chunk", [16, 32, 64])
@pytest.mark.parametrize("T", [1, 63, 100, 130])
def test_chunked_equals_recurrent(chunk, T):
    a = _inputs(T=T, seed=T + chunk)
    o, S = R.recurrent(**a)
    oc, Sc = R.chunked(**a, chunk=chunk)
    np.testing.assert_allclose(oc, o, rtol=1e-4, atol=1e-5)
    assert np.linalg.norm(Sc - S) / np.linalg.norm(S) < 1e-5


def test_chunked_varlen_equals_recurrent():
    cu = np.array([0, 0, 70, 71, 200])
    a = _inputs(T=200, seed=12, N=4)
    o, S = R.recurrent(**a, cu_seqlens=cu)
    oc, Sc = R.chunked(**a, cu_seqlens=cu)
    np.testing.assert_allclose(oc, o, rtol=1e-4, atol=1e-5)
    assert np.linalg.norm(Sc - S) / np.linalg.norm(S) < 1e-5


@pytest.mark.parametrize("kind", ["chunk", "recurrent"])
@pytest.mark.parametrize("shape", [(2, 100, 2, 4, 64, 64), (1, 77, 1, 2, 128, 128), (1, 65, 4, 4, 128, 64)])
def test_c_port_equals_numpy_oracle(kind, shape):
    B, T, Hqk, Hv, K, V = shape
    a = _inputs(B=B, T=T, Hqk=Hqk, Hv=Hv, K=K, V=V, seed=sum(shape))
    a = {kk: (None if x is None else x.astype(np.float32)) for kk, x in a.items()}
    o, S = R.recurrent(**a)
    oc, Sc = coracle.run(kind, **a, threads=4)
    np.testing.assert_allclose(oc, o, rtol=2e-4, atol=2e-5)
    assert np.linalg.norm(Sc - S) / np.linalg.norm(S) < 2e-5


def test_c_port_varlen_and_l2norm():
    cu = np.array([0, 5, 5, 130, 131], np.int32)
    a = _inputs(T=131, seed=13, N=4, K=64, V=64, unit=False)
    a = {kk: x.astype(np.float32) for kk, x in a.items()}
    o, S = R.recurrent(**a, cu_seqlens=cu, use_qk_l2norm=True)
    for kind in ("chunk", "recurrent"):
        oc, Sc = coracle.run(kind, **a, cu_seqlens=cu, use_qk_l2norm=True, threads=3)
        np.testing.assert_allclose(oc, o, rtol=2e-4, atol=2e-5)
        assert np.linalg.norm(Sc - S) / np.linalg.norm(S) < 2e-5


# ------------------------------------------------------------ mutation checks

def _mutant(kind):
    """Copies of the token recurrence with one plausible mistake planted."""
    def run(q, k, v, g, beta, initial_state=None):
        B, T, Hqk, K = q.shape
        Hv, V = v.shape[2:]
        S = np.zeros((B, Hv, K, V)) if initial_state is None else initial_state.copy()
        o = np.zeros((B, T, Hv, V))
        for t in range(T):
            for h in range(Hv):
                hq = (h % Hqk) if kind == "gqa_modulo" else h // (Hv // Hqk)
                qt, kt = q[0, t, hq], k[0, t, hq]
                eg = np.exp(g[0, t, h])
                St = S[0, h]
                if kind == "decay_after_read":
                    d = beta[0, t, h] * (v[0, t, h] - kt @ St)
                    St = eg * St
                else:
                    St = eg * St
                    d = beta[0, t, h] * (v[0, t, h] - kt @ St)
                    if kind == "beta_dropped":
                        d = v[0, t, h] - kt @ St
                if kind == "transposed":
                    St = St + np.outer(d, kt) if K == V else St
                else:
                    St = St + np.outer(kt, d)
                S[0, h] = St
                o[0, t, h] = K ** -0.5 * (qt @ St)
        return o, S
    return run


@pytest.mark.parametrize("kind", ["decay_after_read", "beta_dropped", "transposed", "gqa_modulo"])
def test_planted_mistakes_are_caught(kind):
    """Each mutant disagrees with a closed form / invariant checked above."""
    a = _inputs(T=6, seed=14, K=8, V=8, Hqk=2, Hv=4, h0=True)
    mut = _mutant(kind)
    om, Sm = mut(a["q"], a["k"], a["v"], a["g"], a["beta"], a["initial_state"])
    o, S = R.recurrent(**a)
    assert not (np.allclose(om, o, atol=1e-8) and np.allclose(Sm, S, atol=1e-8))
    if kind == "transposed":   # caught by the single-token outer-product form
        b = _inputs(T=1, seed=15, K=8, V=8, h0=False)
        _, S1 = mut(b["q"], b["k"], b["v"], b["g"], b["beta"])
        kk, vv, bb = b["k"][0, 0, 0], b["v"][0, 0, 0], b["beta"][0, 0, 0]
        assert not np.allclose(S1[0, 0], bb * np.outer(kk, vv))
    if kind == "decay_after_read":   # caught by the per-step retrieval identity
        b = _inputs(T=2, seed=16, K=8, V=8, h0=True)
        _, Sp = mut(*(b[n][:, :1] for n in ("q", "k", "v", "g", "beta")), b["initial_state"])
        _, Sc = mut(*(b[n] for n in ("q", "k", "v", "g", "beta")), b["initial_state"])
        kt = b["k"][0, 1, 0]
        bt, gt = b["beta"][0, 1, 0], b["g"][0, 1, 0]
        want = (1 - bt) * np.exp(gt) * (kt @ Sp[0, 0]) + bt * b["v"][0, 1, 0]
        assert not np.allclose(kt @ Sc[0, 0], want, atol=1e-10)
