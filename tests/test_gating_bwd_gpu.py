"""GPU parity of the gating backward (gdn_gating_bwd, fused_gdn_gating_bwd) and
of training through the fused gating (chunk_gated_delta_rule_gated under
autograd).

The kernel is checked against oracle/layer_ref.gating_bwd (fp64; pinned in
tests/test_layer_oracle.py against torch's own autograd and finite
differences): da and db to one rounding of their dtype (half a subnormal
step where fp16 values underflow), the per-head sums
dA_log and ddt_bias (fp32 sums of up to 70,000 rows) to 1e-5 of the sum of
their terms' magnitudes plus one rounding of the parameters' dtype.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from avelang_amd import workloads as W
from oracle import layer_ref as LR

pytestmark = pytest.mark.gpu

ULP = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
# half the spacing of the dtype's subnormals (fp16's start at 2^-24; the others' are far below
# any value here)
TINY = {torch.float32: 1e-38, torch.bfloat16: 1e-38, torch.float16: 2.0 ** -25}


def _inputs(dev, rows, H, adt, bdt, pdt, seed, spb=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    a = rng.standard_normal((rows, H)).astype(np.float32) * 3
    if rows:
        a[0, : min(H, 2)] = [30.0 / spb, -30.0][: min(H, 2)]     # threshold branch, tail
    b = rng.standard_normal((rows, H)).astype(np.float32) * 3
    A_log = np.log(rng.uniform(0.5, 8.0, H)).astype(np.float32)
    dt = (rng.standard_normal(H) * 0.5).astype(np.float32)
    dg = rng.standard_normal((rows, H)).astype(np.float32)
    dbeta = rng.standard_normal((rows, H)).astype(np.float32)
    to = lambda x, d: torch.from_numpy(x).to(dev, d)  # noqa: E731
    return to(A_log, pdt), to(a, adt), to(b, bdt), to(dt, pdt), to(dg, torch.float32), \
        to(dbeta, torch.float32)


def _check(got, ts, spb, spt):
    A_log, a, b, dt, dg, dbeta = (t.float().cpu().numpy() for t in ts)
    ref = LR.gating_bwd(A_log, a, b, dt, dg, dbeta, spb, spt)
    dA_r, da_r, db_r, ddt_r = ref
    dA, da, db, ddt = got
    # elementwise: one rounding of the output dtype (plus fp32 math)
    for x, r, what in ((da, da_r, "da"), (db, db_r, "db")):
        u = ULP[x.dtype]
        err = np.abs(x.float().cpu().numpy() - r)
        bound = u * np.abs(r) + 1e-6 * np.abs(r) + TINY[x.dtype]
        assert (err <= bound).all(), f"{what}: max excess {(err - bound).max():.3e}"
    # per-head sums
    g, _ = LR.gating(A_log, a, b, dt, spb, spt)
    mag_A = np.abs(dg * g).sum(axis=0)
    mag_dt = np.abs(da_r).sum(axis=0)
    for x, r, mag, what in ((dA, dA_r, mag_A, "dA_log"), (ddt, ddt_r, mag_dt, "ddt_bias")):
        u = ULP[x.dtype]
        err = np.abs(x.float().cpu().numpy() - r)
        bound = 1e-5 * mag + u * np.abs(r) + TINY[x.dtype]
        assert (err <= bound).all(), f"{what}: max excess {(err - bound).max():.3e}"


@pytest.mark.parametrize("rows,H,adt,bdt,pdt", [
    (300, 32, torch.bfloat16, torch.bfloat16, torch.float32),
    (8192, 32, torch.bfloat16, torch.bfloat16, torch.float32),     # config 1's gating
    (70000, 32, torch.float32, torch.float32, torch.float32),      # > 64 rows per block
    (257, 7, torch.float16, torch.float32, torch.bfloat16),
    (65, 256, torch.bfloat16, torch.float16, torch.float16),
    (1, 1, torch.float32, torch.bfloat16, torch.float32),
])
def test_gating_bwd_matches_oracle(rocm_device, rows, H, adt, bdt, pdt):
    from avelang_amd import fused_gdn_gating_bwd
    ts = _inputs(rocm_device, rows, H, adt, bdt, pdt, seed=rows + H)
    got = fused_gdn_gating_bwd(*ts)
    torch.cuda.synchronize()
    assert got[1].dtype == adt and got[2].dtype == bdt
    assert got[0].dtype == pdt and got[3].dtype == pdt
    _check(got, ts, 1.0, 20.0)


def test_gating_bwd_softplus_parameters(rocm_device):
    from avelang_amd import fused_gdn_gating_bwd
    ts = _inputs(rocm_device, 500, 16, torch.bfloat16, torch.bfloat16, torch.float32, seed=5,
                 spb=2.0)
    got = fused_gdn_gating_bwd(*ts, beta=2.0, threshold=5.0)
    _check(got, ts, 2.0, 5.0)


def test_gating_bwd_empty_rows_give_zero_parameter_grads(rocm_device):
    from avelang_amd import fused_gdn_gating_bwd
    ts = _inputs(rocm_device, 0, 8, torch.bfloat16, torch.bfloat16, torch.float32, seed=1)
    dA, da, db, ddt = fused_gdn_gating_bwd(*ts)
    assert da.numel() == 0 and db.numel() == 0
    assert torch.equal(dA, torch.zeros_like(dA)) and torch.equal(ddt, torch.zeros_like(ddt))


def test_gating_bwd_without_dbeta(rocm_device):
    from avelang_amd import fused_gdn_gating_bwd
    A_log, a, b, dt, dg, dbeta = _inputs(rocm_device, 100, 8, torch.bfloat16, torch.bfloat16,
                                         torch.float32, seed=2)
    full = fused_gdn_gating_bwd(A_log, a, b, dt, dg, dbeta)
    part = fused_gdn_gating_bwd(A_log, a, b, dt, dg, None)
    assert part[2] is None
    for x, y in zip((full[0], full[1], full[3]), (part[0], part[1], part[3])):
        assert torch.equal(x, y)


def test_gating_bwd_deterministic(rocm_device):
    from avelang_amd import fused_gdn_gating_bwd
    ts = _inputs(rocm_device, 70000, 32, torch.bfloat16, torch.bfloat16, torch.float32, seed=3)
    x = fused_gdn_gating_bwd(*ts)
    y = fused_gdn_gating_bwd(*ts)
    for u, v in zip(x, y):
        assert torch.equal(u, v)


def test_fused_gdn_gating_autograd(rocm_device):
    """fused_gdn_gating under autograd: its gradients are fused_gdn_gating_bwd's, and agree
    with torch's autograd of the layer's expression in fp32."""
    from avelang_amd import fused_gdn_gating, fused_gdn_gating_bwd
    A_log, a, b, dt, dg, dbeta = _inputs(rocm_device, 1000, 32, torch.float32, torch.float32,
                                         torch.float32, seed=4)
    leaves = [t.clone().requires_grad_() for t in (A_log, a, b, dt)]
    g, beta = fused_gdn_gating(*leaves)
    ((g * dg).sum() + (beta * dbeta).sum()).backward()
    want = fused_gdn_gating_bwd(A_log, a, b, dt, dg, dbeta)
    for leaf, w in zip(leaves, want):
        assert torch.equal(leaf.grad, w)
    ref = [t.clone().requires_grad_() for t in (A_log, a, b, dt)]
    g_t = -torch.exp(ref[0]) * F.softplus(ref[1] + ref[3])
    ((g_t * dg).sum() + (torch.sigmoid(ref[2]) * dbeta).sum()).backward()
    for leaf, r in zip(leaves, ref):
        torch.testing.assert_close(leaf.grad, r.grad, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("save", [True, False])
def test_chunk_gated_training_matches_composition(rocm_device, save):
    """Training through chunk_gated_delta_rule_gated equals the layer's composition (torch-op
    gating in fp32 under autograd, then chunk_gated_delta_rule): every gradient within 1e-3
    (both backwards run gdn_chunk_bwd; they differ only in the last bits of g and beta)."""
    from avelang_amd import chunk_gated_delta_rule, chunk_gated_delta_rule_gated
    cu = np.array([0, 333, 334, 1000], dtype=np.int32)
    wl = W.make(1, 1000, 16, 32, 128, 128, seed=91, h0_scale=0.01, cu_seqlens=cu)
    t = wl.torch(rocm_device)
    A_log, a, b, dt, _, _ = _inputs(rocm_device, 1000, 32, torch.bfloat16, torch.bfloat16,
                                    torch.float32, seed=92)
    a, b = a[None], b[None]
    gen = torch.Generator(device=rocm_device).manual_seed(93)
    do = torch.randn(t["v"].shape, generator=gen, device=rocm_device).to(torch.bfloat16)
    dht = 0.01 * torch.randn(t["initial_state"].shape, generator=gen, device=rocm_device)

    def run(fused):
        leaves = {n: x.clone().requires_grad_() for n, x in
                  (("q", t["q"]), ("k", t["k"]), ("v", t["v"]), ("a", a), ("b", b),
                   ("A_log", A_log), ("dt", dt), ("h0", t["initial_state"]))}
        kw = dict(initial_state=leaves["h0"], output_final_state=True,
                  cu_seqlens=t["cu_seqlens"], save_for_backward=save)
        if fused:
            o, ht = chunk_gated_delta_rule_gated(leaves["q"], leaves["k"], leaves["v"],
                                                 leaves["a"], leaves["b"], leaves["A_log"],
                                                 leaves["dt"], **kw)
        else:
            g = -torch.exp(leaves["A_log"].float()) * F.softplus(leaves["a"].float()
                                                                 + leaves["dt"])
            beta = torch.sigmoid(leaves["b"].float())
            o, ht = chunk_gated_delta_rule(leaves["q"], leaves["k"], leaves["v"], g, beta, **kw)
        ((o.float() * do.float()).sum() + (ht * dht).sum()).backward()
        return o, {n: x.grad for n, x in leaves.items()}

    o1, g1 = run(True)
    o2, g2 = run(False)
    torch.cuda.synchronize()
    assert (o1.float() - o2.float()).abs().max().item() <= 2 ** -7 * o2.float().abs().max().item()
    for n in g1:
        assert g1[n] is not None and g1[n].dtype == g2[n].dtype, n
        x, y = g1[n].float(), g2[n].float()
        fro = ((x - y).norm() / y.norm()).item()
        print(f"gated training {n}: relative Frobenius difference {fro:.2e}", flush=True)
        assert fro <= 1e-3, (n, fro)
