"""GPU parity of the gating fused into the core (gdn_chunk_fwd_gating,
gdn_recurrent_fwd_gating).

The fused paths form g and beta inside the prep / decode kernels with the
same device function the standalone gating kernel uses, so they must equal
fused_gdn_gating followed by the core bit for bit; and, independently, the
CPU oracle (oracle/layer_ref.gating in fp64, then the C chunked / recurrent
oracle) within the prefill tolerances.
"""
import numpy as np
import pytest
import torch

from avelang_amd import workloads as W
from oracle import cpu as oracle
from oracle import layer_ref as LR

pytestmark = pytest.mark.gpu

O_TOL = 2e-2
S_FRO = 1e-3


def _gates(dev, B, T, Hv, seed, pdtype=torch.float32, adtype=torch.bfloat16):
    rng = np.random.Generator(np.random.PCG64(seed))
    a = torch.from_numpy(rng.standard_normal((B, T, Hv), dtype=np.float32)).to(dev, adtype)
    b = torch.from_numpy(rng.standard_normal((B, T, Hv), dtype=np.float32)).to(dev, adtype)
    # A = exp(A_log) in [0.5, 8): the range of Qwen3-Next's initialisation
    # (uniform(0, 16)) without its smallest values
    A_log = torch.from_numpy(np.log(rng.uniform(0.5, 8.0, Hv)).astype(np.float32)).to(dev, pdtype)
    dt_bias = torch.from_numpy(rng.standard_normal(Hv).astype(np.float32) * 0.5).to(dev, pdtype)
    return a, b, A_log, dt_bias


def _fro(x, ref):
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-30))


def _oracle(kind, wl, a, b, A_log, dt_bias, l2=False):
    g, beta = LR.gating(A_log.float().cpu().numpy(), a.float().cpu().numpy(),
                        b.float().cpu().numpy(), dt_bias.float().cpu().numpy())
    n = wl.numpy()
    n["g"], n["beta"] = g.astype(np.float32), beta.astype(np.float32)
    if l2:   # the kernels round the normalised q, k to bf16 (FLA's l2norm pass)
        nrm = lambda x: x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)  # noqa: E731
        n["q"], n["k"] = W._bf16_round(nrm(n["q"])), W._bf16_round(nrm(n["k"]))
    return oracle.run(kind, **n)


@pytest.mark.parametrize("l2,pdt", [(False, torch.float32), (True, torch.bfloat16)])
def test_chunk_fused_gating_equals_two_step(rocm_device, l2, pdt):
    from avelang_amd import (chunk_gated_delta_rule, chunk_gated_delta_rule_gated,
                             fused_gdn_gating)
    cu = np.array([0, 333, 334, 1000], dtype=np.int32)
    wl = W.make(1, 1000, 16, 32, 128, 128, seed=81, h0_scale=0.01, cu_seqlens=cu,
                l2norm=not l2)
    t = wl.torch(rocm_device)
    a, b, A_log, dt_bias = _gates(rocm_device, 1, 1000, 32, 82, pdtype=pdt)
    g, beta = fused_gdn_gating(A_log, a, b, dt_bias)
    kw = dict(initial_state=t["initial_state"], output_final_state=True,
              cu_seqlens=t["cu_seqlens"], use_qk_l2norm_in_kernel=l2)
    o1, s1 = chunk_gated_delta_rule(t["q"], t["k"], t["v"], g, beta, **kw)
    o2, s2 = chunk_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log, dt_bias, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o_ref, s_ref = _oracle("chunk", wl, a, b, A_log, dt_bias, l2)
    err = np.abs(o2.float().cpu().numpy() - o_ref)
    assert (err <= O_TOL + O_TOL * np.abs(o_ref)).all(), f"o max err {err.max():.3e}"
    assert _fro(s2.cpu().numpy(), s_ref) <= S_FRO


def test_decode_fused_gating_equals_two_step(rocm_device):
    from avelang_amd import (fused_gdn_gating, fused_recurrent_gated_delta_rule,
                             fused_recurrent_gated_delta_rule_gated)
    wl = W.make(64, 1, 16, 32, 128, 128, seed=83, h0_scale=0.05)
    t = wl.torch(rocm_device)
    a, b, A_log, dt_bias = _gates(rocm_device, 64, 1, 32, 84)
    g, beta = fused_gdn_gating(A_log, a, b, dt_bias)
    s1 = t["initial_state"].clone()
    s2 = t["initial_state"].clone()
    o1, _ = fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], g, beta,
                                             initial_state=s1, output_final_state=True)
    o2, _ = fused_recurrent_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log,
                                                   dt_bias, initial_state=s2,
                                                   output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o_ref, s_ref = _oracle("recurrent", wl, a, b, A_log, dt_bias)
    err = np.abs(o2.float().cpu().numpy() - o_ref)
    assert (err <= O_TOL + O_TOL * np.abs(o_ref)).all(), f"o max err {err.max():.3e}"
    assert _fro(s2.cpu().numpy(), s_ref) <= S_FRO


def test_decode_fused_gating_slot_pool(rocm_device):
    from avelang_amd import (fused_gdn_gating, fused_recurrent_gated_delta_rule,
                             fused_recurrent_gated_delta_rule_gated)
    N, slots = 16, 40
    wl = W.make(N, 2, 2, 4, 128, 128, seed=85, h0_scale=0.0)
    t = wl.torch(rocm_device)
    a, b, A_log, dt_bias = _gates(rocm_device, N, 2, 4, 86, adtype=torch.float16)
    g, beta = fused_gdn_gating(A_log, a, b, dt_bias)
    idx = torch.randperm(slots)[:N].to(torch.int32)
    idx[3] = -1                                    # a padding sequence
    pool = torch.randn((slots, 4, 128, 128), device=rocm_device) * 0.05
    p1, p2 = pool.clone(), pool.clone()
    o1, _ = fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], g, beta,
                                             initial_state=p1, output_final_state=True,
                                             ssm_state_indices=idx.to(rocm_device))
    o2, _ = fused_recurrent_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log,
                                                   dt_bias, initial_state=p2,
                                                   output_final_state=True,
                                                   ssm_state_indices=idx.to(rocm_device))
    torch.cuda.synchronize()
    live = torch.ones(N, dtype=torch.bool)
    live[3] = False
    assert torch.equal(o1[live], o2[live]) and torch.equal(p1, p2)


@pytest.mark.parametrize("l2", [False, True])
def test_decode_fused_gating_varlen(rocm_device, l2):
    """Packed sequences of 3, 0, 1, 6, 0 and 7 tokens: a sequence's first-token
    gate is loaded a tile ahead and formed by one wave, later tokens' gates in
    place; empty sequences keep their state."""
    from avelang_amd import (fused_gdn_gating, fused_recurrent_gated_delta_rule,
                             fused_recurrent_gated_delta_rule_gated)
    cu = np.array([0, 3, 3, 4, 10, 10, 17], dtype=np.int32)
    wl = W.make(1, 17, 4, 8, 128, 128, seed=87, h0_scale=0.05, cu_seqlens=cu, l2norm=not l2)
    t = wl.torch(rocm_device)
    a, b, A_log, dt_bias = _gates(rocm_device, 1, 17, 8, 88)
    g, beta = fused_gdn_gating(A_log, a, b, dt_bias)
    s1 = t["initial_state"].clone()
    s2 = t["initial_state"].clone()
    kw = dict(output_final_state=True, cu_seqlens=t["cu_seqlens"], use_qk_l2norm_in_kernel=l2)
    o1, _ = fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], g, beta, initial_state=s1,
                                             **kw)
    o2, _ = fused_recurrent_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log, dt_bias,
                                                   initial_state=s2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    # the decode kernel normalises q, k in fp32 inside its dot products (no
    # bf16 rounding of the normalised rows), as the oracle's own l2norm does
    gg, bb = LR.gating(A_log.float().cpu().numpy(), a.float().cpu().numpy(),
                       b.float().cpu().numpy(), dt_bias.float().cpu().numpy())
    n = wl.numpy()
    n["g"], n["beta"] = gg.astype(np.float32), bb.astype(np.float32)
    o_ref, s_ref = oracle.run("recurrent", **n, use_qk_l2norm=l2)
    err = np.abs(o2.float().cpu().numpy() - o_ref)
    assert (err <= O_TOL + O_TOL * np.abs(o_ref)).all(), f"o max err {err.max():.3e}"
    assert _fro(s2.cpu().numpy(), s_ref) <= S_FRO
