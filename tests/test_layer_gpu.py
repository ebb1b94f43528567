"""GPU parity of the layer operators (csrc/gdn_layer.hip, slot-indexed decode)
against the numpy oracle (oracle/layer_ref.py) on the same inputs.

Every call goes through the C ABI (avelang_amd.layer_ops / the recurrent
operator -> libgdn.so).  Tolerances: fp32 results rtol 1e-5; results
rounded to bf16 within one bf16 rounding step (rel 2^-7) of the oracle
evaluated on the same bf16 inputs; the GDN core as in test_gdn_gpu.py
(o atol = rtol = 2e-2, state relative Frobenius <= 1e-3); state copies
(conv states) bit-exact.
"""
import numpy as np
import pytest
import torch

from avelang_amd import layer_ops as L
from avelang_amd import fused_recurrent_gated_delta_rule, chunk_gated_delta_rule
from oracle import gdn_ref as R
from oracle import layer_ref as LR

pytestmark = pytest.mark.gpu

BF_REL = 2.0 ** -7


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _close_lowp(got, ref, what, rel=BF_REL, floor=1e-2):
    got = _np(got)
    err = np.abs(got - ref)
    bad = err > rel * np.maximum(np.abs(ref), floor)
    assert not bad.any(), (f"{what}: {bad.sum()} / {bad.size} entries off, "
                           f"max abs err {err.max():.3e}")


def _rand(shape, dev, dtype=torch.bfloat16, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(dev)


# ---------------------------------------------------------------- gating ----
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_gating(rocm_device, dt):
    dev = rocm_device
    T, H = 4096, 32
    a = _rand((1, T, H), dev, dt, 3.0, 1)
    b = _rand((1, T, H), dev, dt, 3.0, 2)
    a[0, 0, :3] = torch.tensor([25.0, -40.0, 19.5], dtype=dt)
    A_log = torch.log(torch.linspace(0.5, 16, H)).to(dev)
    dt_bias = _rand((H,), dev, torch.float32, 1.0, 3)
    g, beta = L.fused_gdn_gating(A_log, a, b, dt_bias)
    torch.cuda.synchronize()
    g_ref, b_ref = LR.gating(_np(A_log), _np(a), _np(b), _np(dt_bias))
    np.testing.assert_allclose(_np(g), g_ref, rtol=1e-5, atol=1e-30)
    np.testing.assert_allclose(_np(beta), b_ref, rtol=1e-5, atol=1e-7)
    assert g.dtype == torch.float32 and g.shape == a.shape


def test_gating_feeds_chunk_path(rocm_device):
    """Gates made on the GPU drive the prefill exactly like host-made ones."""
    dev = rocm_device
    B, T, Hqk, Hv, K = 1, 96, 2, 4, 128
    q = L.l2norm_fwd(_rand((B, T, Hqk, K), dev, seed=4))
    k = L.l2norm_fwd(_rand((B, T, Hqk, K), dev, seed=5))
    v = _rand((B, T, Hv, K), dev, seed=6)
    a, b = _rand((B, T, Hv), dev, seed=7), _rand((B, T, Hv), dev, seed=8)
    A_log, dt_bias = torch.zeros(Hv, device=dev), torch.zeros(Hv, device=dev)
    g, beta = L.fused_gdn_gating(A_log, a, b, dt_bias)
    o, s = chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True)
    torch.cuda.synchronize()
    g_ref, b_ref = LR.gating(0 * _np(A_log), _np(a), _np(b), 0 * _np(dt_bias))
    o_ref, s_ref = R.recurrent(_np(q), _np(k), _np(v), g_ref, b_ref)
    o_g = _np(o)
    assert np.all(np.abs(o_g - o_ref) <= 2e-2 + 2e-2 * np.abs(o_ref))
    assert np.linalg.norm(_np(s) - s_ref) / np.linalg.norm(s_ref) <= 1e-3


# -------------------------------------------------------------- l2norm ----
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_l2norm(rocm_device, D, dt):
    x = _rand((3, 77, 5, D), rocm_device, dt, 2.0, D)
    y = L.l2norm_fwd(x)
    torch.cuda.synchronize()
    ref = R.l2norm(_np(x))
    if dt == torch.float32:
        np.testing.assert_allclose(_np(y), ref, rtol=1e-5, atol=1e-7)
    else:
        _close_lowp(y, ref, f"l2norm D={D}")
    yi = x.clone()
    L.l2norm_fwd(yi, out=yi)                     # in place
    torch.cuda.synchronize()
    assert torch.equal(yi, y)


# ---------------------------------------------------------- causal conv ----
def _conv_case(dev, B, D, T, W, dt, layout, seed=0):
    base = _rand((B, T, D), dev, dt, 1.0, seed)
    if layout == "channel_last":                  # the layer's [B, T, D] memory
        x = base.transpose(1, 2)
    elif layout == "time_contiguous":
        x = base.transpose(1, 2).contiguous()
    else:                                         # a strided slice: generic kernel
        x = _rand((B, 2 * D, T + 3), dev, dt, 1.0, seed)[:, ::2, 3:]
    w = _rand((D, W), dev, torch.float32, 0.5, seed + 1)
    bias = _rand((D,), dev, torch.float32, 0.5, seed + 2)
    return x, w, bias


@pytest.mark.parametrize("layout", ["channel_last", "time_contiguous", "strided"])
@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("silu", [False, True])
def test_conv_fn_layouts(rocm_device, layout, W, silu):
    x, w, bias = _conv_case(rocm_device, 2, 64, 301, W, torch.bfloat16, layout, seed=W)
    out = L.causal_conv1d_fn(x, w, bias, activation="silu" if silu else None)
    torch.cuda.synchronize()
    assert out.stride() == x.stride() or layout == "strided"
    ref, _ = LR.causal_conv1d(_np(x), _np(w), _np(bias), silu=silu)
    _close_lowp(out, ref, f"conv {layout} W={W}")


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_conv_fn_dtypes(rocm_device, dt):
    x, w, bias = _conv_case(rocm_device, 1, 128, 257, 4, dt, "channel_last", seed=9)
    out = L.causal_conv1d_fn(x, w.to(dt), bias.to(dt), activation="silu")
    torch.cuda.synchronize()
    ref, _ = LR.causal_conv1d(_np(x), _np(w.to(dt)), _np(bias.to(dt)), silu=True)
    if dt == torch.float32:
        np.testing.assert_allclose(_np(out), ref, rtol=1e-5, atol=1e-5)
    else:
        _close_lowp(out, ref, "conv f16", rel=2.0 ** -10, floor=1e-3)


def test_conv_fn_seq_idx_and_states(rocm_device):
    dev = rocm_device
    lens = [37, 1, 90, 3, 129]
    T = sum(lens)
    x, w, bias = _conv_case(dev, 1, 128, T, 4, torch.bfloat16, "channel_last", seed=12)
    sq = torch.tensor(np.concatenate([np.full(n, i) for i, n in enumerate(lens)])[None],
                      dtype=torch.int32, device=dev)
    out = L.causal_conv1d_fn(x, w, bias, seq_idx=sq, activation="silu")
    torch.cuda.synchronize()
    ref, _ = LR.causal_conv1d(_np(x), _np(w), _np(bias), seq_idx=_np(sq), silu=True)
    _close_lowp(out, ref, "conv seq_idx")
    for layout in ("channel_last", "strided"):
        x, w, bias = _conv_case(dev, 2, 64, 50, 4, torch.bfloat16, layout, seed=13)
        init = _rand((2, 64, 3), dev, seed=14)
        out, fin = L.causal_conv1d_fn(x, w, bias, initial_states=init,
                                      return_final_states=True, activation="silu")
        torch.cuda.synchronize()
        ref, fref = LR.causal_conv1d(_np(x), _np(w), _np(bias), initial_states=_np(init),
                                     silu=True)
        _close_lowp(out, ref, f"conv init {layout}")
        np.testing.assert_array_equal(_np(fin), fref)
    # rows shorter than the window and empty rows
    for T in (2, 0):
        x, w, bias = _conv_case(dev, 2, 64, T, 4, torch.bfloat16, "channel_last", seed=15)
        init = _rand((2, 64, 3), dev, seed=16)
        out, fin = L.causal_conv1d_fn(x, w, bias, initial_states=init, return_final_states=True)
        torch.cuda.synchronize()
        _, fref = LR.causal_conv1d(_np(x), _np(w), _np(bias), initial_states=_np(init))
        np.testing.assert_array_equal(_np(fin), fref)


def test_conv_fn_qwen3_next_shape(rocm_device):
    """Layer shape (conv_dim 8192, T 8192, channel-last bf16): oracle on 96 channels."""
    dev = rocm_device
    D, T = 8192, 8192
    x, w, bias = _conv_case(dev, 1, D, T, 4, torch.bfloat16, "channel_last", seed=21)
    out = L.causal_conv1d_fn(x, w, None, activation="silu")
    torch.cuda.synchronize()
    ch = np.sort(np.random.default_rng(0).choice(D, 96, replace=False))
    chs = torch.tensor(ch, device=dev)
    ref, _ = LR.causal_conv1d(_np(x[:, chs]), _np(w[chs]), silu=True)
    _close_lowp(out[:, chs], ref, "conv qwen3-next shape")


# ------------------------------------------------------ causal conv update ----
@pytest.mark.parametrize("S,L_new", [(3, 1), (3, 4), (4, 1), (6, 3)])
def test_conv_update_matches_prefill(rocm_device, S, L_new):
    """Prefill of [0, t) then decode updates == one prefill (split-resume)."""
    dev = rocm_device
    B, D, T, W = 3, 256, 24, 4
    x, w, bias = _conv_case(dev, B, D, T, W, torch.bfloat16, "channel_last", seed=30 + S)
    full = L.causal_conv1d_fn(x, w, bias, activation="silu")
    t = 10
    state = torch.zeros((B, D, S), dtype=x.dtype, device=dev)
    state[:, :, S - (W - 1):] = x[:, :, t - (W - 1):t]
    state[:, :, :S - (W - 1)] = x[:, :, t - S:t - (W - 1)]
    outs = []
    for a in range(t, T, L_new):
        e = min(a + L_new, T)
        step = x[:, :, a:e]
        outs.append(L.causal_conv1d_update(step if e - a > 1 else step[:, :, 0], state, w, bias,
                                           activation="silu"))
    torch.cuda.synchronize()
    got = torch.cat([o if o.dim() == 3 else o.unsqueeze(-1) for o in outs], dim=2)
    _close_lowp(got, _np(full[:, :, t:]), f"conv update S={S} L={L_new}")
    assert torch.equal(state, x[:, :, T - S:].contiguous())


def test_conv_update_slots_and_padding(rocm_device):
    dev = rocm_device
    B, D, S, slots = 4, 8192, 3, 7
    x = _rand((B, D), dev, seed=40)
    pool = _rand((slots, D, S), dev, seed=41)
    before = pool.clone()
    w = _rand((D, 4), dev, torch.bfloat16, 0.5, 42)
    idx = torch.tensor([6, -1, 2, 9], dtype=torch.int32, device=dev)   # -1 / 9: padding rows
    out = L.causal_conv1d_update(x, pool, w, None, activation="silu", conv_state_indices=idx)
    torch.cuda.synchronize()
    ref, new = LR.causal_conv1d_update(_np(x)[:, :, None], _np(before), _np(w),
                                       indices=[6, -1, 2, 9], silu=True)
    _close_lowp(out[[0, 2]], ref[[0, 2], :, 0], "conv update slots")
    np.testing.assert_array_equal(_np(pool), new)
    assert torch.equal(pool[[0, 1, 3, 4, 5]], before[[0, 1, 3, 4, 5]])


# ----------------------------------------------------------- gated norm ----
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_rms_norm_gated(rocm_device, D, wdt):
    dev = rocm_device
    x = _rand((5, 333, D), dev, seed=D)
    z = _rand((5, 333, D), dev, scale=2.0, seed=D + 1)
    w = (1 + 0.1 * _rand((D,), dev, torch.float32, seed=D + 2)).to(wdt)
    out = L.rms_norm_gated(x, z, w, eps=1e-6)
    torch.cuda.synchronize()
    ref = LR.rmsnorm_gated(_np(x), _np(z), _np(w), 1e-6, dtype="bf16",
                           weight_dtype="bf16" if wdt == torch.bfloat16 else "f32")
    got = _np(out)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3)
    assert (rel <= BF_REL + 1e-9).all(), rel.max()
    assert (got == ref).mean() > 0.97


def test_rms_norm_gated_fp32(rocm_device):
    dev = rocm_device
    x = _rand((64, 128), dev, torch.float32, seed=3)
    z = _rand((64, 128), dev, torch.float32, seed=4)
    w = _rand((128,), dev, torch.float32, seed=5)
    out = L.rms_norm_gated(x, z, w)
    torch.cuda.synchronize()
    ref = LR.rmsnorm_gated(_np(x), _np(z), _np(w), dtype="f32", weight_dtype="f32")
    np.testing.assert_allclose(_np(out), ref, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------- slot pools ----
def test_recurrent_state_pool(rocm_device):
    dev = rocm_device
    B, Hqk, Hv, K, V, slots = 5, 2, 4, 128, 128, 9
    q = L.l2norm_fwd(_rand((B, 1, Hqk, K), dev, seed=50))
    k = L.l2norm_fwd(_rand((B, 1, Hqk, K), dev, seed=51))
    v = _rand((B, 1, Hv, V), dev, seed=52)
    g = -0.1 * torch.rand((B, 1, Hv), device=dev)
    beta = torch.rand((B, 1, Hv), device=dev)
    pool = 0.01 * torch.randn((slots, Hv, K, V), device=dev)
    before = pool.clone()
    idx = torch.tensor([7, 0, -1, 3, 12], dtype=torch.int32, device=dev)
    o = torch.full_like(v, 7.0)
    o, ret = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool,
                                              output_final_state=True,
                                              ssm_state_indices=idx, out=o)
    torch.cuda.synchronize()
    assert ret is pool
    o_ref, pool_ref = LR.recurrent_indexed(_np(q), _np(k), _np(v), _np(g), _np(beta),
                                           _np(before), [7, 0, -1, 3, 12])
    live = [0, 1, 3]
    got = _np(o)
    assert np.all(np.abs(got[live] - o_ref[live]) <= 2e-2 + 2e-2 * np.abs(o_ref[live]))
    assert (got[[2, 4]] == 7.0).all()                        # padding rows untouched
    for s in (7, 0, 3):
        fro = np.linalg.norm(_np(pool[s]) - pool_ref[s]) / np.linalg.norm(pool_ref[s])
        assert fro <= 1e-3
    assert torch.equal(pool[[1, 2, 4, 5, 6, 8]], before[[1, 2, 4, 5, 6, 8]])
    # the identity map reproduces the plain in-place decode bit for bit
    p1, p2 = before[:B].clone(), before[:B].clone()
    o1, _ = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=p1,
                                             output_final_state=True,
                                             ssm_state_indices=torch.arange(B, dtype=torch.int32,
                                                                            device=dev))
    o2, _ = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=p2,
                                             output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(p1, p2)


# ---------------------------------------------------- layer composition ----
def test_layer_prefill_then_decode(rocm_device):
    """conv -> split -> gating -> GDN (l2norm in kernel) -> gated norm, then one
    decode step through conv update + slot-indexed recurrence, against the
    oracle chain evaluated on the same bf16 intermediate roundings."""
    dev = rocm_device
    T, Hqk, Hv, K = 150, 2, 4, 128
    kd, vd = Hqk * K, Hv * K
    D = 2 * kd + vd
    mixed = _rand((1, T + 1, D), dev, seed=60)
    w = _rand((D, 4), dev, torch.bfloat16, 0.5, 61)
    a, b = _rand((1, T + 1, Hv), dev, seed=62), _rand((1, T + 1, Hv), dev, seed=63)
    A_log = torch.log(torch.linspace(1, 8, Hv)).to(dev)
    dt_bias = _rand((Hv,), dev, torch.float32, 0.5, 64)
    z = _rand((1, T + 1, Hv, K), dev, seed=65)
    nw = (1 + 0.1 * _rand((K,), dev, torch.float32, seed=66)).to(torch.bfloat16)

    def split(c):
        q = c[..., :kd].reshape(*c.shape[:-1], Hqk, K)
        k = c[..., kd:2 * kd].reshape(*c.shape[:-1], Hqk, K)
        v = c[..., 2 * kd:].reshape(*c.shape[:-1], Hv, K)
        return q, k, v

    # prefill of the first T tokens; conv state = last 3 inputs
    conv, fin = L.causal_conv1d_fn(mixed[:, :T].transpose(1, 2), w, None,
                                   return_final_states=True, activation="silu")
    q, k, v = split(conv.transpose(1, 2))
    g, beta = L.fused_gdn_gating(A_log, a[:, :T], b[:, :T], dt_bias)
    o, S = chunk_gated_delta_rule(q.contiguous(), k.contiguous(), v.contiguous(), g, beta,
                                  output_final_state=True, use_qk_l2norm_in_kernel=True)
    y = L.rms_norm_gated(o, z[:, :T], nw)
    # decode of token T: state pool of 3 slots, this sequence in slot 2
    conv_pool = torch.zeros((3, D, 3), dtype=torch.bfloat16, device=dev)
    conv_pool[2] = fin[0]
    ssm_pool = torch.zeros((3, Hv, K, K), device=dev)
    ssm_pool[2] = S[0]
    idx = torch.tensor([2], dtype=torch.int32, device=dev)
    c1 = L.causal_conv1d_update(mixed[:, T], conv_pool, w, None, activation="silu",
                                conv_state_indices=idx)
    q1, k1, v1 = split(c1.unsqueeze(1))
    g1, b1 = L.fused_gdn_gating(A_log, a[:, T:], b[:, T:], dt_bias)
    o1, _ = fused_recurrent_gated_delta_rule(q1.contiguous(), k1.contiguous(), v1.contiguous(),
                                             g1, b1, initial_state=ssm_pool,
                                             output_final_state=True,
                                             use_qk_l2norm_in_kernel=True,
                                             ssm_state_indices=idx)
    y1 = L.rms_norm_gated(o1, z[:, T:], nw)
    torch.cuda.synchronize()

    # oracle chain over all T + 1 tokens, rounding where the GPU path stores bf16:
    # the prefill rounds the normalised q, k to bf16, the decode kernel
    # normalises them in fp32
    c_ref, _ = LR.causal_conv1d(_np(mixed).transpose(0, 2, 1), _np(w), silu=True)
    c_ref = LR.bf16_round(c_ref.astype(np.float32)).astype(np.float64).transpose(0, 2, 1)
    qr, kr, vr = (t.numpy() for t in split(torch.from_numpy(c_ref)))
    qn, kn = R.l2norm(qr), R.l2norm(kr)
    qn[:, :T], kn[:, :T] = (LR.bf16_round(t[:, :T].astype(np.float32)).astype(np.float64)
                            for t in (qn, kn))
    g_ref, b_ref = LR.gating(_np(A_log), _np(a), _np(b), _np(dt_bias))
    o_ref, S_ref = R.recurrent(qn, kn, vr, g_ref, b_ref)
    y_ref = LR.rmsnorm_gated(LR.bf16_round(o_ref.astype(np.float32)), _np(z), _np(nw),
                             dtype="bf16", weight_dtype="bf16")
    y_all = np.concatenate([_np(y), _np(y1)], axis=1)
    err = np.abs(y_all - y_ref)
    assert np.all(err <= 2e-2 + 2e-2 * np.abs(y_ref)), err.max()
    fro = np.linalg.norm(_np(ssm_pool[2]) - S_ref[0]) / np.linalg.norm(S_ref[0])
    assert fro <= 1e-3, fro
    np.testing.assert_array_equal(_np(conv_pool[2]), _np(mixed[0, T - 2:T + 1].T))
