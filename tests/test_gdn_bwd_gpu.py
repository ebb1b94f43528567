"""GPU parity of the chunked backward (gdn_chunk_bwd) against the fp64 oracle.

Every test calls the HIP path through the C ABI (chunk_gated_delta_rule_bwd
or torch.autograd through chunk_gated_delta_rule -> libgdn.so) and compares
with oracle/gdn_bwd_ref.py (chunk-level backward in fp64, pinned against
finite differences and the per-token backward in tests/test_oracle_bwd.py)
on the same seeded inputs: the bf16 values the GPU reads, upcast.

Tolerances (written here, the north star states none for gradients): the
relative Frobenius error of dq, dk, dv, dg and dbeta <= 1e-2 (the gradient
kernel forms its products from bf16 operands with fp32 accumulation; an fp64
emulation of those roundings gives ~2e-3), and dh0 <= 1e-3, the bar of the
forward's final state (the state-gradient chain carries hi + lo bf16 splits
as the forward chain does).
"""
import numpy as np
import pytest
import torch

from avelang_amd import workloads as W
from oracle import gdn_bwd_ref as RB
from oracle import gdn_ref as R

pytestmark = pytest.mark.gpu

G_FRO = 1e-2
H_FRO = 1e-3


def _np(t):
    return t.detach().double().cpu().numpy()


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _grad_inputs(wl, seed, dht_scale=0.01):
    d = wl.dims
    rng = np.random.Generator(np.random.PCG64(seed + 101))
    do = W._bf16_round(rng.standard_normal((d["B"], d["T"], d["Hv"], d["V"]), dtype=np.float32))
    dht = None
    if dht_scale:
        dht = (dht_scale * rng.standard_normal((d["N"], d["Hv"], d["K"], d["V"]),
                                               dtype=np.float32)).astype(np.float32)
    return do, dht


def _gpu_bwd(wl, do, dht, dev, l2=False, scale=None):
    from avelang_amd import chunk_gated_delta_rule_bwd
    t = wl.torch(dev)
    dq, dk, dv, dg, db, dh0 = chunk_gated_delta_rule_bwd(
        t["q"], t["k"], t["v"], t["g"], t["beta"],
        torch.from_numpy(do).to(device=dev, dtype=torch.bfloat16),
        None if dht is None else torch.from_numpy(dht).to(dev),
        scale=scale, initial_state=t["initial_state"], cu_seqlens=t["cu_seqlens"],
        use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    return dict(dq=dq, dk=dk, dv=dv, dg=dg, dbeta=db, dh0=dh0)


def _check(got, ref, what, has_h0=True):
    errs = {}
    for name in ("dq", "dk", "dv", "dg", "dbeta"):
        g = _np(got[name])
        assert np.isfinite(g).all(), f"{what}: {name} has non-finite values"
        errs[name] = _rel(g, ref[name])
    if has_h0:
        errs["dh0"] = _rel(_np(got["dh0"]), ref["dh0"])
    print(f"{what}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        tol = H_FRO if name == "dh0" else G_FRO
        assert e <= tol, f"{what}: {name} relative Frobenius error {e:.3e} > {tol}"
    return errs


def _case(dev, B, T, Hqk, Hv, K, V, seed=0, cu=None, h0_scale=0.01, dht_scale=0.01,
          l2=False, decay=0.1, what=""):
    wl = W.make(B, T, Hqk, Hv, K, V, seed=seed, h0_scale=h0_scale, cu_seqlens=cu, decay=decay,
                l2norm=not l2)
    do, dht = _grad_inputs(wl, seed, dht_scale)
    a = wl.numpy()
    if l2:
        # the operator normalises q, k and rounds them to bf16 before use (as the
        # forward does); the reference runs on those rounded rows and then
        # differentiates through the normalisation of the raw rows
        qn, kn = (W._bf16_round(R.l2norm(a[x].astype(np.float32))) for x in ("q", "k"))
        ref = RB.chunked_bwd(qn, kn, a["v"], a["g"], a["beta"], do, dht,
                             initial_state=a["initial_state"], cu_seqlens=a["cu_seqlens"])
        ref["dq"] = RB.l2norm_bwd(a["q"].astype(np.float64), ref["dq"])
        ref["dk"] = RB.l2norm_bwd(a["k"].astype(np.float64), ref["dk"])
    else:
        ref = RB.chunked_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                             initial_state=a["initial_state"], cu_seqlens=a["cu_seqlens"])
    got = _gpu_bwd(wl, do, dht, dev, l2=l2)
    return _check(got, ref, what or f"B{B} T{T} {Hqk}/{Hv} K{K} V{V}",
                  has_h0=a["initial_state"] is not None)


@pytest.mark.parametrize("T", [64, 200])
def test_bwd_small(rocm_device, T):
    _case(rocm_device, 1, T, 2, 4, 128, 128, seed=T, what=f"small T={T}")


def test_bwd_cfg0_shape(rocm_device):
    """BASELINE config 0 shape (K = V = 64, 4 heads, zero initial state)."""
    _case(rocm_device, 1, 256, 4, 4, 64, 64, seed=3, h0_scale=0.0, dht_scale=0.0, what="cfg0")


@pytest.mark.parametrize("K,V", [(64, 64), (64, 128), (128, 64)])
def test_bwd_head_sizes(rocm_device, K, V):
    _case(rocm_device, 1, 130, 2, 4, K, V, seed=K + V, what=f"K{K} V{V}")


@pytest.mark.parametrize("G", [1, 4])
def test_bwd_gqa_ratio(rocm_device, G):
    _case(rocm_device, 1, 190, 2, 2 * G, 128, 128, seed=10 + G, what=f"GQA {G}")


def test_bwd_batch(rocm_device):
    _case(rocm_device, 3, 100, 2, 4, 128, 128, seed=21, what="B=3")


def test_bwd_varlen_with_empty(rocm_device):
    cu = np.array([0, 0, 70, 71, 200, 200, 329], dtype=np.int32)
    _case(rocm_device, 1, 329, 2, 4, 128, 128, seed=22, cu=cu, what="varlen")


def test_bwd_l2norm(rocm_device):
    _case(rocm_device, 1, 150, 2, 4, 128, 128, seed=23, l2=True, what="l2norm")


def test_bwd_l2norm_many_items(rocm_device):
    """use_qk_l2norm with more (chunk, qk-head) items (150 x 4 = 600) than the gradient kernel
    has resident workgroups, so that each workgroup goes through its item loop several times."""
    _case(rocm_device, 1, 9600, 4, 8, 128, 128, seed=26, l2=True, what="l2norm 600 items")


def test_bwd_no_dht_no_h0(rocm_device):
    _case(rocm_device, 1, 128, 2, 4, 128, 128, seed=24, h0_scale=0.0, dht_scale=0.0,
          what="no h0 / dht")


def test_bwd_long_slow_decay(rocm_device):
    """cfg4's slower decay over 32 chunks: long-range state gradients."""
    _case(rocm_device, 1, 2048, 2, 4, 128, 128, seed=25, decay=0.01, what="T2048 decay .01")


def test_bwd_cfg1_shape(rocm_device):
    """Config 1 in full: T = 8192, 16 qk-heads -> 32 v-heads, K = V = 128."""
    wl = W.config("cfg1_prefill_qwen3next", seed=0)
    do, dht = _grad_inputs(wl, 0)
    a = wl.numpy()
    ref = RB.chunked_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                         initial_state=a["initial_state"])
    got = _gpu_bwd(wl, do, dht, rocm_device)
    _check(got, ref, "cfg1")


def test_autograd_matches_bwd(rocm_device):
    """torch.autograd through chunk_gated_delta_rule == chunk_gated_delta_rule_bwd."""
    from avelang_amd import chunk_gated_delta_rule
    wl = W.make(1, 150, 2, 4, 128, 128, seed=30)
    do, dht = _grad_inputs(wl, 30)
    t = wl.torch(rocm_device)
    leaves = {n: t[n].clone().requires_grad_(True)
              for n in ("q", "k", "v", "g", "beta", "initial_state")}
    o, ht = chunk_gated_delta_rule(leaves["q"], leaves["k"], leaves["v"], leaves["g"],
                                   leaves["beta"], initial_state=leaves["initial_state"],
                                   output_final_state=True)
    dO = torch.from_numpy(do).to(device=rocm_device, dtype=torch.bfloat16)
    dH = torch.from_numpy(dht).to(rocm_device)
    ((o.float() * dO.float()).sum() + (ht * dH).sum()).backward()
    got = _gpu_bwd(wl, do, dht, rocm_device)
    for n, key in (("q", "dq"), ("k", "dk"), ("v", "dv"), ("g", "dg"), ("beta", "dbeta"),
                   ("initial_state", "dh0")):
        a = leaves[n].grad
        assert a is not None, n
        assert torch.equal(a.float(), got[key].float()), f"autograd {n} differs from the bwd call"


def test_bwd_linear_in_output_gradients(rocm_device):
    """No oracle: the gradients are linear in (dO, dht), and every step of the backward commutes
    with doubling (fp16 and bf16 roundings, MFMA products and fp32 sums of doubled operands are
    the doubled results) except where an fp16 operand of the reverse chain falls below fp16's
    normal range (|x| < 2^-14, an absolute rounding step of 2^-24).  So doubling dO and dht
    doubles dh0 (fp32, straight from the reverse chain) to ~1e-6 and the other gradients, formed
    from the chain's bf16 saves, to within a bf16 rounding (config 1's heads, T = 1000)."""
    wl = W.make(1, 1000, 16, 32, 128, 128, seed=31, h0_scale=0.01)
    do, dht = _grad_inputs(wl, 31)
    a = _gpu_bwd(wl, do, dht, rocm_device)
    b = _gpu_bwd(wl, 2 * do, 2 * dht, rocm_device)
    for name in a:
        want = 2 * a[name].float()
        fro = ((b[name].float() - want).norm() / want.norm()).item()
        print(f"doubling {name}: relative Frobenius deviation {fro:.2e}", flush=True)
        assert fro < (1e-5 if name == "dh0" else 2 ** -8), (name, fro)


def test_bwd_deterministic(rocm_device):
    wl = W.make(1, 300, 2, 4, 128, 128, seed=31)
    do, dht = _grad_inputs(wl, 31)
    a = _gpu_bwd(wl, do, dht, rocm_device)
    b = _gpu_bwd(wl, do, dht, rocm_device)
    for key in a:
        assert torch.equal(a[key], b[key]), key


def test_training_forward_matches_forward(rocm_device):
    """gdn_chunk_fwd_save gives gdn_chunk_fwd's o and final state, bitwise."""
    from avelang_amd import chunk_gated_delta_rule, chunk_gated_delta_rule_fwd_save
    cu = np.array([0, 70, 71, 230], dtype=np.int32)
    for l2 in (False, True):
        wl = W.make(1, 230, 2, 4, 128, 128, seed=40, cu_seqlens=cu, l2norm=not l2)
        t = wl.torch(rocm_device)
        kw = dict(initial_state=t["initial_state"], output_final_state=True,
                  cu_seqlens=t["cu_seqlens"], use_qk_l2norm_in_kernel=l2)
        o1, s1 = chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"], **kw)
        o2, s2, _ = chunk_gated_delta_rule_fwd_save(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                                    **kw)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(s1, s2), f"l2norm={l2}"


@pytest.mark.parametrize("l2", [False, True])
def test_saved_backward_equals_recomputed(rocm_device, l2):
    """The backward from a training forward's workspace == the recomputing backward."""
    from avelang_amd import chunk_gated_delta_rule_bwd, chunk_gated_delta_rule_fwd_save
    cu = np.array([0, 0, 100, 163, 300], dtype=np.int32)
    wl = W.make(1, 300, 2, 4, 128, 128, seed=41, cu_seqlens=cu, l2norm=not l2)
    do, dht = _grad_inputs(wl, 41)
    t = wl.torch(rocm_device)
    _, _, ws = chunk_gated_delta_rule_fwd_save(
        t["q"], t["k"], t["v"], t["g"], t["beta"], initial_state=t["initial_state"],
        output_final_state=True, cu_seqlens=t["cu_seqlens"], use_qk_l2norm_in_kernel=l2)
    args = (t["q"], t["k"], t["v"], t["g"], t["beta"],
            torch.from_numpy(do).to(device=rocm_device, dtype=torch.bfloat16),
            torch.from_numpy(dht).to(rocm_device))
    kw = dict(initial_state=t["initial_state"], cu_seqlens=t["cu_seqlens"],
              use_qk_l2norm_in_kernel=l2)
    a = chunk_gated_delta_rule_bwd(*args, workspace=ws, saved=True, **kw)
    b = chunk_gated_delta_rule_bwd(*args, **kw)
    torch.cuda.synchronize()
    for name, x, y in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), a, b):
        assert torch.equal(x, y), name


def test_autograd_without_saved_forward(rocm_device, monkeypatch):
    """SAVE_FORWARD_FOR_BACKWARD = False (recompute) gives the same gradients."""
    from avelang_amd import chunk_gated_delta_rule
    from avelang_amd import gated_delta_rule as GDR
    wl = W.make(1, 150, 2, 4, 128, 128, seed=42)
    do, _ = _grad_inputs(wl, 42)
    dO = torch.from_numpy(do).to(device=rocm_device, dtype=torch.bfloat16)
    grads = []
    for flag in (True, False):
        monkeypatch.setattr(GDR, "SAVE_FORWARD_FOR_BACKWARD", flag)
        t = wl.torch(rocm_device)
        leaves = [t[n].clone().requires_grad_(True) for n in ("q", "k", "v", "g", "beta")]
        o, _ = chunk_gated_delta_rule(*leaves, initial_state=t["initial_state"])
        (o.float() * dO.float()).sum().backward()
        grads.append([x.grad for x in leaves])
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    # and per call, against the module default (True here)
    t = wl.torch(rocm_device)
    leaves = [t[n].clone().requires_grad_(True) for n in ("q", "k", "v", "g", "beta")]
    o, _ = chunk_gated_delta_rule(*leaves, initial_state=t["initial_state"],
                                  save_for_backward=False)
    (o.float() * dO.float()).sum().backward()
    for a, x in zip(grads[0], leaves):
        assert torch.equal(a, x.grad)


def test_bwd_varlen_many_sequences(rocm_device):
    """Config 3's structure (packed sequences of lengths U[128, 4096], seeded) at 8 sequences
    and 2 qk-heads -> 4 v-heads, so the fp64 oracle stays fast."""
    cu = W.varlen_cu_seqlens(8, 128, 4096, seed=3)
    _case(rocm_device, 1, int(cu[-1]), 2, 4, 128, 128, seed=50, cu=cu, what="varlen 8 seqs")


def test_bwd_long_context(rocm_device):
    """Config 4's slow decay over a 16384-token sequence (256 chunks), 1 qk-head -> 2 v-heads."""
    _case(rocm_device, 1, 16384, 1, 2, 128, 128, seed=51, decay=0.01, what="T16384 decay .01")


def test_bwd_two_tiles_per_workgroup(rocm_device):
    """Enough chains for two V tiles per workgroup in the recomputed forward
    (chain with saves): parity against the oracle, and sequence 0's
    gradients equal, bit for bit, those of the sequence run alone."""
    from avelang_amd import chunk_gated_delta_rule_bwd
    cus = torch.cuda.get_device_properties(rocm_device).multi_processor_count
    Hqk, Hv, K, V = 2, 4, 128, 128
    B = -(-2 * cus // (Hv * (V // 16)))
    wl = W.make(B, 96, Hqk, Hv, K, V, seed=94, h0_scale=0.01)
    do, dht = _grad_inputs(wl, 94)
    a = wl.numpy()
    ref = RB.chunked_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, dht,
                         initial_state=a["initial_state"])
    got = _gpu_bwd(wl, do, dht, rocm_device)
    _check(got, ref, f"two tiles B{B}")
    t = wl.torch(rocm_device)
    one = chunk_gated_delta_rule_bwd(
        t["q"][:1], t["k"][:1], t["v"][:1], t["g"][:1], t["beta"][:1],
        torch.from_numpy(do[:1]).to(device=rocm_device, dtype=torch.bfloat16),
        torch.from_numpy(dht[:1]).to(rocm_device), initial_state=t["initial_state"][:1])
    torch.cuda.synchronize()
    for name, x in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), one):
        assert torch.equal(got[name][:1], x), name
