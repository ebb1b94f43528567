"""Pinning checks for the layer-operator oracle (oracle/layer_ref.py; CPU only).

Each oracle function is checked against something it does not share code
with:

  library routines  torch (CPU) softplus / sigmoid / exp, torch.nn.functional
                    conv1d with groups = channels, torch's own bf16 / fp16
                    arithmetic for the rounding steps of the gated norm
  closed forms      delta kernels (identity, pure delay), SiLU(0) = 0, a
                    constant row normalises to 1, softplus's threshold branch
  invariants        split-resume (prefill then decode updates == one prefill),
                    packed sequences == independent rows, slot pools ==
                    gathering / scattering the plain recurrence
  mutation checks   planted mistakes (no left padding, window reversed,
                    state shifted the wrong way, gate applied before the norm)
                    each fail one of the above
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_ref as R
from oracle import layer_ref as LR

RNG = np.random.default_rng


# ---------------------------------------------------------------- gating ----
def test_gating_matches_torch_library_routines():
    rng = RNG(1)
    H = 8
    a = rng.standard_normal((64, H)) * 4
    a[0, :4] = [25.0, 19.9, -30.0, 0.0]          # threshold branch and tails
    b = rng.standard_normal((64, H)) * 3
    A_log = np.log(rng.uniform(0.5, 16, H))
    dt = rng.standard_normal(H)
    g, beta = LR.gating(A_log, a, b, dt)
    ta = torch.tensor(a) + torch.tensor(dt)
    g_t = -torch.exp(torch.tensor(A_log)) * F.softplus(ta, beta=1.0, threshold=20.0)
    np.testing.assert_allclose(g, g_t.numpy(), rtol=1e-12, atol=0)
    np.testing.assert_allclose(beta, torch.sigmoid(torch.tensor(b)).numpy(), rtol=1e-12)


def test_gating_softplus_parameters():
    a = np.array([[3.0, -2.0, 10.5]])
    g, _ = LR.gating(np.zeros(3), a, np.zeros((1, 3)), np.zeros(3), sp_beta=2.0, threshold=20.0)
    ref = -F.softplus(torch.tensor(a), beta=2.0, threshold=20.0).numpy()
    np.testing.assert_allclose(g, ref, rtol=1e-12)
    # beyond the threshold softplus is the identity
    g, _ = LR.gating(np.zeros(1), np.array([[21.0]]), np.zeros((1, 1)), np.zeros(1))
    assert g[0, 0] == -21.0


def _gating_grad_inputs(seed, shape=(3, 5, 8)):
    rng = RNG(seed)
    H = shape[-1]
    a = rng.standard_normal(shape) * 4
    a.flat[:3] = [25.0, -30.0, 0.0]              # threshold branch and tails
    return (np.log(rng.uniform(0.5, 16, H)), a, rng.standard_normal(shape) * 3,
            rng.standard_normal(H), rng.standard_normal(shape), rng.standard_normal(shape))


@pytest.mark.parametrize("spb,spt", [(1.0, 20.0), (2.0, 5.0)])
def test_gating_bwd_matches_torch_autograd(spb, spt):
    """gating_bwd against torch's own autograd of the layer's expression (float64, CPU)."""
    A_log, a, b, dt, dg, dbeta = _gating_grad_inputs(3)
    ts = [torch.tensor(x, requires_grad=True) for x in (A_log, a, b, dt)]
    g = -torch.exp(ts[0]) * F.softplus(ts[1] + ts[3], beta=spb, threshold=spt)
    beta = torch.sigmoid(ts[2])
    ((g * torch.tensor(dg)).sum() + (beta * torch.tensor(dbeta)).sum()).backward()
    got = LR.gating_bwd(A_log, a, b, dt, dg, dbeta, spb, spt)
    for x, t in zip(got, ts):
        np.testing.assert_allclose(x, t.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_gating_bwd_finite_differences():
    """gating_bwd against central differences of gating itself (away from the threshold)."""
    A_log, a, b, dt, dg, dbeta = _gating_grad_inputs(4, shape=(4, 6))
    a.flat[:3] = [2.0, -3.0, 0.5]
    got = LR.gating_bwd(A_log, a, b, dt, dg, dbeta)

    def loss(A_, a_, b_, d_):
        g, beta = LR.gating(A_, a_, b_, d_)
        return (g * dg).sum() + (beta * dbeta).sum()

    args = [A_log, a, b, dt]
    eps = 1e-6
    for which, grad in zip(range(4), got):
        fd = np.zeros_like(args[which])
        for idx in np.ndindex(args[which].shape):
            hi = [x.copy() for x in args]
            lo = [x.copy() for x in args]
            hi[which][idx] += eps
            lo[which][idx] -= eps
            fd[idx] = (loss(*hi) - loss(*lo)) / (2 * eps)
        np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-8)


def test_gating_bwd_mutations_caught():
    """A softplus derivative at the wrong beta, or a dropped exp(A_log), fails the check."""
    A_log, a, b, dt, dg, dbeta = _gating_grad_inputs(5)
    ts = [torch.tensor(x, requires_grad=True) for x in (A_log, a, b, dt)]
    g = -torch.exp(ts[0]) * F.softplus(ts[1] + ts[3], beta=2.0, threshold=20.0)
    ((g * torch.tensor(dg)).sum() + (torch.sigmoid(ts[2]) * torch.tensor(dbeta)).sum()).backward()
    good = LR.gating_bwd(A_log, a, b, dt, dg, dbeta, 2.0, 20.0)
    np.testing.assert_allclose(good[1], ts[1].grad.numpy(), rtol=1e-12)
    wrong_scale = LR.gating_bwd(A_log, a, b, dt, dg, dbeta, 1.0, 20.0)[1]
    assert not np.allclose(wrong_scale, ts[1].grad.numpy(), rtol=1e-6)
    no_exp = LR.gating_bwd(np.zeros_like(A_log), a, b, dt, dg, dbeta, 2.0, 20.0)[1]
    assert not np.allclose(no_exp, ts[1].grad.numpy(), rtol=1e-6)


# ---------------------------------------------------------- causal conv ----
def _conv_inputs(B=2, D=6, T=11, W=4, seed=0):
    rng = RNG(seed)
    return (rng.standard_normal((B, D, T)), rng.standard_normal((D, W)),
            rng.standard_normal(D))


@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("silu", [False, True])
def test_conv_matches_torch_conv1d(W, silu):
    x, w, b = _conv_inputs(W=W, seed=W)
    out, fin = LR.causal_conv1d(x, w, b, silu=silu)
    ref = F.conv1d(torch.tensor(x), torch.tensor(w).unsqueeze(1), torch.tensor(b),
                   padding=W - 1, groups=x.shape[1])[..., :x.shape[2]]
    if silu:
        ref = F.silu(ref)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(fin, x[:, :, -(W - 1):])


def test_conv_delta_kernels():
    x, _, _ = _conv_inputs(W=4)
    ident = np.zeros((x.shape[1], 4)); ident[:, 3] = 1
    out, _ = LR.causal_conv1d(x, ident)
    np.testing.assert_array_equal(out, x)
    delay = np.zeros((x.shape[1], 4)); delay[:, 0] = 1         # x[t-3], zero padded
    out, _ = LR.causal_conv1d(x, delay)
    np.testing.assert_array_equal(out[:, :, 3:], x[:, :, :-3])
    assert not out[:, :, :3].any()


def test_conv_initial_states_equal_concatenation():
    x, w, b = _conv_inputs(T=9)
    full = np.concatenate([RNG(5).standard_normal((2, 6, 3)), x], axis=2)
    out_full, fin_full = LR.causal_conv1d(full, w, b)
    out, fin = LR.causal_conv1d(x, w, b, initial_states=full[:, :, :3])
    np.testing.assert_allclose(out, out_full[:, :, 3:], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(fin, fin_full)


def test_conv_short_rows_final_states_come_from_initial_states():
    x, w, _ = _conv_inputs(T=1)
    init = RNG(6).standard_normal((2, 6, 3))
    _, fin = LR.causal_conv1d(x, w, initial_states=init)
    np.testing.assert_array_equal(fin, np.concatenate([init[:, :, 1:], x], axis=2))


def test_conv_seq_idx_equals_independent_rows():
    rng = RNG(7)
    lens = [5, 1, 7, 3]
    T = sum(lens)
    x = rng.standard_normal((1, 4, T))
    w = rng.standard_normal((4, 4))
    sq = np.concatenate([np.full(n, i) for i, n in enumerate(lens)])[None]
    out, _ = LR.causal_conv1d(x, w, seq_idx=sq, silu=True)
    s = 0
    for n in lens:
        ref, _ = LR.causal_conv1d(x[:, :, s:s + n], w, silu=True)
        np.testing.assert_allclose(out[:, :, s:s + n], ref, rtol=1e-12, atol=1e-12)
        s += n


@pytest.mark.parametrize("S", [3, 5])
def test_conv_update_split_resume(S):
    """Prefill of [0, t) then decode updates of the rest == one prefill."""
    x, w, b = _conv_inputs(T=13, seed=3)
    W = 4
    ref, _ = LR.causal_conv1d(x, w, b, silu=True)
    t = 6
    _, fin = LR.causal_conv1d(x[:, :, :t], w, b, silu=True)
    state = np.zeros((x.shape[0], x.shape[1], S))
    state[:, :, S - (W - 1):] = fin
    if S > W - 1:                                   # older inputs kept in a longer state
        state[:, :, :S - (W - 1)] = x[:, :, t - S:t - (W - 1)]
    outs = []
    for a, e in [(6, 7), (7, 10), (10, 13)]:        # 1 token, then 3, then 3
        o, state = LR.causal_conv1d_update(x[:, :, a:e], state, w, b, silu=True)
        outs.append(o)
    np.testing.assert_allclose(np.concatenate(outs, axis=2), ref[:, :, t:], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(state, x[:, :, 13 - S:])


def test_conv_update_slots_and_padding():
    rng = RNG(9)
    x = rng.standard_normal((3, 4, 1))
    pool = rng.standard_normal((5, 4, 3))
    w = rng.standard_normal((4, 4))
    out, new = LR.causal_conv1d_update(x, pool, w, indices=[4, -1, 0])
    o4, s4 = LR.causal_conv1d_update(x[0:1], pool[4:5], w)
    o0, s0 = LR.causal_conv1d_update(x[2:3], pool[0:1], w)
    np.testing.assert_array_equal(out[0], o4[0])
    np.testing.assert_array_equal(out[2], o0[0])
    assert np.isnan(out[1]).all()
    np.testing.assert_array_equal(new[4], s4[0])
    np.testing.assert_array_equal(new[0], s0[0])
    np.testing.assert_array_equal(new[[1, 2, 3]], pool[[1, 2, 3]])


def _planted_conv_no_padding(x, w):
    # mistake: "valid" convolution shifted to the start (no causal left padding)
    W = w.shape[1]
    out = np.zeros_like(x)
    for j in range(W):
        sl = x[:, :, j:]
        out[:, :, :sl.shape[2]] += w[:, j][None, :, None] * sl
    return out


def _planted_conv_reversed(x, w):
    out, _ = LR.causal_conv1d(x, w[:, ::-1])
    return out


@pytest.mark.parametrize("planted", [_planted_conv_no_padding, _planted_conv_reversed])
def test_conv_mutations_caught(planted):
    x, w, _ = _conv_inputs(W=4, seed=11)
    ref = F.conv1d(torch.tensor(x), torch.tensor(w).unsqueeze(1), padding=3,
                   groups=x.shape[1])[..., :x.shape[2]].numpy()
    assert not np.allclose(planted(x, w), ref, atol=1e-6)


def test_conv_update_mutation_caught():
    """State shifted the wrong way (new inputs dropped) breaks split-resume."""
    x, w, _ = _conv_inputs(T=8, seed=4)
    ref, _ = LR.causal_conv1d(x, w)
    _, fin = LR.causal_conv1d(x[:, :, :5], w)
    state = fin.copy()
    outs = []
    for t in range(5, 8):
        win = np.concatenate([state, x[:, :, t:t + 1]], axis=2)
        outs.append((win * w[None]).sum(-1, keepdims=True))
        state = win[:, :, :3]                         # wrong end kept
    assert not np.allclose(np.concatenate(outs, 2), ref[:, :, 5:], atol=1e-6)


# ----------------------------------------------------------- gated norm ----
def _torch_gated_norm(x, z, w, eps, dt):
    """The norm's arithmetic in torch's own low-precision types (library rounding)."""
    xt, zt, wt = (torch.tensor(a, dtype=torch.float32).to(dt) for a in (x, z, w))
    h = xt.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    h = wt * h.to(dt)
    h = h * F.silu(zt.to(torch.float32))
    return h.to(dt).to(torch.float32).numpy()


@pytest.mark.parametrize("dt,kind", [(torch.bfloat16, "bf16"), (torch.float16, "f16")])
def test_gated_norm_rounding_steps_match_torch(dt, kind):
    rng = RNG(2)
    rnd = LR.bf16_round if kind == "bf16" else LR.f16_round
    x = rnd(rng.standard_normal((200, 128)).astype(np.float32))
    z = rnd(rng.standard_normal((200, 128)).astype(np.float32) * 2)
    w = rnd((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    ours = LR.rmsnorm_gated(x, z, w, 1e-6, dtype=kind, weight_dtype=kind)
    ref = _torch_gated_norm(x, z, w, 1e-6, dt)
    ulp = 2.0 ** -7 if kind == "bf16" else 2.0 ** -10
    diff = np.abs(ours - ref) / np.maximum(np.abs(ref), 1e-3)
    assert (diff <= ulp + 1e-9).all()              # at most one rounding step apart
    assert (ours == ref).mean() > 0.97


def test_gated_norm_closed_forms():
    x = np.full((3, 64), 2.5, np.float32)
    z = np.zeros((3, 64), np.float32)
    w = np.ones(64, np.float32)
    assert not LR.rmsnorm_gated(x, z, w).any()                     # silu(0) = 0
    z = np.full((3, 64), 30.0, np.float32)                          # silu(z) ~ z
    out = LR.rmsnorm_gated(x, z, w, eps=0.0)
    np.testing.assert_allclose(out, 30.0, rtol=1e-6)                # constant row -> 1


def test_gated_norm_mutation_caught():
    """Gate applied before the norm (norm_before_gate=False) differs."""
    rng = RNG(8)
    x = rng.standard_normal((10, 64)).astype(np.float32)
    z = rng.standard_normal((10, 64)).astype(np.float32)
    w = np.ones(64, np.float32)
    ours = LR.rmsnorm_gated(x, z, w)
    xz = x * (z / (1 + np.exp(-z)))
    planted = xz / np.sqrt((xz ** 2).mean(-1, keepdims=True) + 1e-6)
    assert not np.allclose(ours, planted, atol=1e-3)


# --------------------------------------------------------- slot pools ----
def test_recurrent_indexed_equals_gather_scatter():
    rng = RNG(4)
    B, T, Hqk, Hv, K, V = 3, 5, 1, 2, 8, 8
    q = rng.standard_normal((B, T, Hqk, K)); k = rng.standard_normal((B, T, Hqk, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, V))
    g = -0.1 * rng.random((B, T, Hv)); beta = rng.random((B, T, Hv))
    pool = rng.standard_normal((6, Hv, K, V))
    idx = [5, -1, 2]
    o, new = LR.recurrent_indexed(q, k, v, g, beta, pool, idx)
    o_ref, S = R.recurrent(q[[0, 2]], k[[0, 2]], v[[0, 2]], g[[0, 2]], beta[[0, 2]],
                           initial_state=pool[[5, 2]])
    np.testing.assert_allclose(o[[0, 2]], o_ref, rtol=1e-12)
    assert np.isnan(o[1]).all()
    np.testing.assert_allclose(new[[5, 2]], S, rtol=1e-12)
    np.testing.assert_array_equal(new[[0, 1, 3, 4]], pool[[0, 1, 3, 4]])
    # identity map == the plain recurrence over the first B slots
    o2, new2 = LR.recurrent_indexed(q, k, v, g, beta, pool[:3], [0, 1, 2])
    o3, S3 = R.recurrent(q, k, v, g, beta, initial_state=pool[:3])
    np.testing.assert_allclose(o2, o3, rtol=1e-12)
    np.testing.assert_allclose(new2, S3, rtol=1e-12)


def test_bf16_round_matches_torch():
    x = RNG(3).standard_normal(10000).astype(np.float32) * 100
    x[:4] = [0.0, -0.0, 1e-30, 3.0e38]
    ref = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(LR.bf16_round(x), ref)
