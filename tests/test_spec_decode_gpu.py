"""GPU parity of speculative-decoding steps (per-token states in a slot pool).

fused_recurrent_gated_delta_rule with a 2-D ssm_state_indices [N, S] writes
the state after every token of a multi-token (draft-verification) step into
its own slot; num_accepted_tokens picks the slot a later step starts from.
Checked against the fp32 CPU oracle run over token prefixes, at config 2's
head shape (16 qk-heads -> 32 v-heads, K = V = 128).
"""
import numpy as np
import pytest
import torch

from avelang_amd import workloads as W
from oracle import cpu as oracle

pytestmark = pytest.mark.gpu

O_TOL = 2e-2
S_FRO = 1e-3


def _fro(x, ref):
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-30))


def _prefix(a, t):
    """Oracle inputs restricted to the first t tokens of every sequence."""
    return {key: (val[:, :t] if key in ("q", "k", "v", "g", "beta") else val)
            for key, val in a.items()}


def _spec_step(dev, wl, pool, idx, accepted=None, l2=False):
    from avelang_amd import fused_recurrent_gated_delta_rule
    t = wl.torch(dev)
    o, p = fused_recurrent_gated_delta_rule(
        t["q"], t["k"], t["v"], t["g"], t["beta"], initial_state=pool, output_final_state=True,
        ssm_state_indices=idx, num_accepted_tokens=accepted, use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    assert p.data_ptr() == pool.data_ptr()
    return o


@pytest.mark.parametrize("l2", [False, True])
def test_spec_per_token_states_cfg2_heads(rocm_device, l2):
    """Every per-token state of a 4-token step equals the oracle over that prefix."""
    N, S = 16, 4
    wl = W.make(N, S, 16, 32, 128, 128, seed=31, h0_scale=0.01)
    a = wl.numpy()
    rng = np.random.Generator(np.random.PCG64(7))
    slots = rng.permutation(3 * N * S)[: N * S].astype(np.int32).reshape(N, S)
    pool = torch.zeros((3 * N * S, 32, 128, 128), dtype=torch.float32, device=rocm_device)
    h0 = torch.from_numpy(a["initial_state"]).to(rocm_device)
    pool[torch.from_numpy(slots[:, 0]).long().to(rocm_device)] = h0
    o = _spec_step(rocm_device, wl, pool, torch.from_numpy(slots).to(rocm_device), l2=l2)
    o_ref, _ = oracle.run("recurrent", **a, use_qk_l2norm=l2)
    err = np.abs(o.float().cpu().numpy() - o_ref)
    assert (err <= O_TOL + O_TOL * np.abs(o_ref)).all(), f"o max err {err.max():.3e}"
    pc = pool.cpu().numpy()
    for t in range(1, S + 1):
        _, s_ref = oracle.run("recurrent", **_prefix(a, t), use_qk_l2norm=l2)
        fro = _fro(pc[slots[:, t - 1]], s_ref)
        assert fro <= S_FRO, f"state after token {t}: rel fro {fro:.3e}"


def test_spec_accepted_prefix_rollback(rocm_device):
    """Step 2 starts from the slot of step 1's last accepted draft token: the
    result equals one run over the accepted tokens followed by step 2's."""
    N, S = 16, 4
    w1 = W.make(N, S, 16, 32, 128, 128, seed=41, h0_scale=0.01)
    w2 = W.make(N, S, 16, 32, 128, 128, seed=42, h0_scale=0.0)
    a1, a2 = w1.numpy(), w2.numpy()
    rng = np.random.Generator(np.random.PCG64(8))
    perm = rng.permutation(2 * N * S).astype(np.int32)
    idx1, idx2 = perm[: N * S].reshape(N, S), perm[N * S:].reshape(N, S)
    accepted = rng.integers(1, S + 1, size=N).astype(np.int32)
    dev = rocm_device
    pool = torch.zeros((2 * N * S, 32, 128, 128), dtype=torch.float32, device=dev)
    pool[torch.from_numpy(idx1[:, 0]).long().to(dev)] = torch.from_numpy(a1["initial_state"]).to(dev)
    _spec_step(dev, w1, pool, torch.from_numpy(idx1).to(dev))
    # step 2's table: fresh slots, except that entry accepted[n] - 1 of row n names
    # the slot holding the state after step 1's last accepted token (read first,
    # then overwritten by step 2's state after its token accepted[n] - 1)
    table = idx2.copy()
    table[np.arange(N), accepted - 1] = idx1[np.arange(N), accepted - 1]
    o2 = _spec_step(dev, w2, pool, torch.from_numpy(table).to(dev),
                    accepted=torch.from_numpy(accepted).to(dev))
    pc = pool.cpu().numpy()
    for n in range(N):
        acc = int(accepted[n])
        cat = {key: np.concatenate([a1[key][n:n + 1, :acc], a2[key][n:n + 1]], 1)
               for key in ("q", "k", "v", "g", "beta")}
        o_ref, s_ref = oracle.run("recurrent", **cat,
                                  initial_state=a1["initial_state"][n:n + 1])
        err = np.abs(o2[n].float().cpu().numpy() - o_ref[0, acc:])
        assert (err <= O_TOL + O_TOL * np.abs(o_ref[0, acc:])).all(), f"seq {n}: o {err.max():.3e}"
        fro = _fro(pc[table[n, S - 1]][None], s_ref)
        assert fro <= S_FRO, f"seq {n} (accepted {acc}): final state rel fro {fro:.3e}"


def test_spec_padding_rows_untouched(rocm_device):
    """An initial slot outside the pool (or an accepted count of 0) leaves the
    sequence's outputs and every slot untouched."""
    N, S = 4, 3
    wl = W.make(N, S, 2, 4, 128, 128, seed=51, h0_scale=0.01)
    dev = rocm_device
    pool = torch.randn((N * S + 2, 4, 128, 128), device=dev)
    before = pool.clone()
    idx = torch.arange(N * S, dtype=torch.int32).reshape(N, S)
    idx[1, 0] = -1                                   # padding sequence (no accepted arg)
    from avelang_amd import fused_recurrent_gated_delta_rule
    t = wl.torch(dev)
    o = torch.full_like(t["v"], 7.0)
    fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                     initial_state=pool, output_final_state=True,
                                     ssm_state_indices=idx.to(dev), out=o)
    torch.cuda.synchronize()
    assert torch.equal(pool[idx[1, 1:].long().to(dev)], before[idx[1, 1:].long().to(dev)])
    assert (o[1] == 7.0).all()
    assert not torch.equal(pool[idx[0].long().to(dev)], before[idx[0].long().to(dev)])
    acc = torch.tensor([1, 1, 0, 1], dtype=torch.int32, device=dev)   # 0 = padding
    pool2 = before.clone()
    o = torch.full_like(t["v"], 7.0)
    idx2 = torch.arange(N * S, dtype=torch.int32).reshape(N, S).to(dev)
    fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                     initial_state=pool2, output_final_state=True,
                                     ssm_state_indices=idx2, num_accepted_tokens=acc, out=o)
    torch.cuda.synchronize()
    assert (o[2] == 7.0).all()
    assert torch.equal(pool2[idx2[2].long()], before[idx2[2].long()])


@pytest.mark.parametrize("Hqk,Hv,K,V", [(16, 32, 128, 128), (2, 4, 64, 64)])
def test_spec_packed_drafts_of_mixed_length(rocm_device, Hqk, Hv, K, V):
    """Packed drafts (cu_seqlens) of lengths 3, 0, 6, 1 with a slot row of S = 4: every slot
    a token writes holds the oracle state after that prefix; the 6-token draft's tokens 5 and
    6 (past the row) advance the state without writing any slot; the empty draft writes
    nothing; every slot outside the written ones keeps its contents; o equals the oracle."""
    lens = [3, 0, 6, 1]
    N, S = len(lens), 4
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    wl = W.make(1, int(cu[-1]), Hqk, Hv, K, V, seed=61, h0_scale=0.01, cu_seqlens=cu)
    a = wl.numpy()
    dev = rocm_device
    rng = np.random.Generator(np.random.PCG64(9))
    nslots = 3 * N * S
    idx = rng.permutation(nslots)[: N * S].astype(np.int32).reshape(N, S)
    pool = 0.5 * torch.randn((nslots, Hv, K, V), device=dev)
    pool[torch.from_numpy(idx[:, 0]).long().to(dev)] = torch.from_numpy(a["initial_state"]).to(dev)
    before = pool.clone()
    t = wl.torch(dev)
    from avelang_amd import fused_recurrent_gated_delta_rule
    o, p = fused_recurrent_gated_delta_rule(
        t["q"], t["k"], t["v"], t["g"], t["beta"], initial_state=pool, output_final_state=True,
        cu_seqlens=t["cu_seqlens"], ssm_state_indices=torch.from_numpy(idx).to(dev))
    torch.cuda.synchronize()
    assert p.data_ptr() == pool.data_ptr()
    o_ref, _ = oracle.run("recurrent", **a)
    err = np.abs(o.float().cpu().numpy() - o_ref)
    assert (err <= O_TOL + O_TOL * np.abs(o_ref)).all(), f"o max err {err.max():.3e}"
    pc, bc = pool.cpu().numpy(), before.cpu().numpy()
    written = set()
    for n, L in enumerate(lens):
        seq = {key: a[key][:, cu[n]:cu[n + 1]] for key in ("q", "k", "v", "g", "beta")}
        for tt in range(1, min(L, S) + 1):
            _, s_ref = oracle.run("recurrent", **{key: val[:, :tt] for key, val in seq.items()},
                                  initial_state=a["initial_state"][n:n + 1])
            fro = _fro(pc[idx[n, tt - 1]][None], s_ref)
            assert fro <= S_FRO, f"seq {n} state after token {tt}: rel fro {fro:.3e}"
            written.add(int(idx[n, tt - 1]))
    for sl in range(nslots):
        if sl not in written:
            assert np.array_equal(pc[sl], bc[sl]), f"slot {sl} changed"
