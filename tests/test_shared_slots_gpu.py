"""The device-side guard on shared state slots (gdn_recurrent_fwd_indexed,
gdn_recurrent_fwd_spec, and the fused-gating decode over a pool).

Two sequences that name the same slot of a device-resident table would
advance it from two workgroups at once.  The kernel finds every such
sequence first: each leaves its slots untouched and gets NaN output rows,
and every other sequence's results are bit for bit those of a run in which
the sharers are padding.  A speculative-decoding row may repeat its own
slot, and table entries a sequence never reads or writes do not count.
"""
import numpy as np
import pytest
import torch

from avelang_amd import workloads as W

pytestmark = pytest.mark.gpu


def _decode(dev, wl, pool, idx, out_fill=7.0, **kw):
    from avelang_amd import fused_recurrent_gated_delta_rule
    t = wl.torch(dev)
    o = torch.full_like(t["v"], out_fill)
    fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                     initial_state=pool, output_final_state=True,
                                     cu_seqlens=t.get("cu_seqlens"),
                                     ssm_state_indices=idx.to(dev), out=o, **kw)
    torch.cuda.synchronize()
    return o


def _rows(o, wl, n):
    """Output rows of sequence n ([tokens, Hv, V])."""
    if wl.cu_seqlens is None:
        return o[n]
    cu = wl.cu_seqlens
    return o[0, int(cu[n]):int(cu[n + 1])]


@pytest.mark.parametrize("T", [1, 3])
def test_indexed_shared_slot(rocm_device, T):
    dev = rocm_device
    N, nslots = 6, 9
    wl = W.make(N, T, 16, 32, 128, 128, seed=71, h0_scale=0.01)
    pool = 0.01 * torch.randn((nslots, 32, 128, 128), device=dev)
    before = pool.clone()
    idx = torch.tensor([0, 3, 3, 5, -1, 7], dtype=torch.int32)      # sequences 1, 2 share 3
    o = _decode(dev, wl, pool, idx)
    ref_pool = before.clone()
    o_ref = _decode(dev, wl, ref_pool, torch.tensor([0, -1, -1, 5, -1, 7], dtype=torch.int32))
    for n in (1, 2):
        assert torch.isnan(o[n].float()).all(), n
    assert torch.equal(pool[3], before[3])
    assert (o[4] == 7.0).all()                                       # padding: unwritten
    for n in (0, 3, 5):
        assert torch.equal(o[n], o_ref[n]), n
    assert torch.equal(pool, ref_pool)


def test_indexed_shared_slot_with_fused_gating(rocm_device):
    from avelang_amd import fused_recurrent_gated_delta_rule_gated
    dev = rocm_device
    N, nslots = 4, 6
    wl = W.make(N, 1, 16, 32, 128, 128, seed=72, h0_scale=0.01)
    t = wl.torch(dev)
    gen = torch.Generator(device=dev).manual_seed(73)
    a = torch.randn((N, 1, 32), generator=gen, device=dev).to(torch.bfloat16)
    b = torch.randn((N, 1, 32), generator=gen, device=dev).to(torch.bfloat16)
    A_log = torch.log(torch.rand(32, generator=gen, device=dev) * 7 + 0.5)
    dt = 0.5 * torch.randn(32, generator=gen, device=dev)
    pool = 0.01 * torch.randn((nslots, 32, 128, 128), device=dev)
    before = pool.clone()
    o = torch.full_like(t["v"], 7.0)
    fused_recurrent_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log, dt,
                                           initial_state=pool, output_final_state=True,
                                           ssm_state_indices=torch.tensor(
                                               [2, 4, 2, 1], dtype=torch.int32, device=dev),
                                           out=o)
    torch.cuda.synchronize()
    assert torch.isnan(o[0].float()).all() and torch.isnan(o[2].float()).all()
    assert torch.equal(pool[2], before[2])
    assert not torch.isnan(o[1].float()).any() and not torch.isnan(o[3].float()).any()
    assert not torch.equal(pool[4], before[4])


def test_spec_shared_slot_across_rows(rocm_device):
    dev = rocm_device
    N, S = 4, 3
    wl = W.make(N, S, 16, 32, 128, 128, seed=74, h0_scale=0.01)
    nslots = 16
    pool = 0.01 * torch.randn((nslots, 32, 128, 128), device=dev)
    before = pool.clone()
    idx = torch.tensor([[0, 1, 2],
                        [3, 4, 2],        # slot 2 also row 0's: rows 0 and 1 share
                        [5, 5, 5],        # a row repeating its own slot: allowed
                        [6, 7, 8]], dtype=torch.int32)
    o = _decode(dev, wl, pool, idx)
    ref_idx = idx.clone()
    ref_idx[0, 0] = -1                    # rows 0 and 1 as padding sequences
    ref_idx[1, 0] = -1
    ref_pool = before.clone()
    o_ref = _decode(dev, wl, ref_pool, ref_idx)
    for n in (0, 1):
        assert torch.isnan(o[n].float()).all(), n
    for s in (0, 1, 2, 3, 4):
        assert torch.equal(pool[s], before[s]), s
    for n in (2, 3):
        assert torch.equal(o[n], o_ref[n]), n
        assert not torch.isnan(o[n].float()).any()
    assert torch.equal(pool, ref_pool)


def test_spec_unused_entries_do_not_count(rocm_device):
    """Packed drafts of lengths 1 and 3 (S = 3): row 0's entries past its one token name
    row 1's slots, but row 0 never writes them, so nothing is shared; and a row whose
    accepted count makes it padding touches nothing, whatever its table row holds."""
    dev = rocm_device
    lens = [1, 3, 2]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    wl = W.make(1, int(cu[-1]), 16, 32, 128, 128, seed=75, h0_scale=0.01, cu_seqlens=cu)
    nslots = 12
    pool = 0.01 * torch.randn((nslots, 32, 128, 128), device=dev)
    before = pool.clone()
    idx = torch.tensor([[0, 4, 5],
                        [3, 4, 5],
                        [3, 4, 9]], dtype=torch.int32)
    acc = torch.tensor([1, 1, 0], dtype=torch.int32, device=dev)     # row 2: padding
    o = _decode(dev, wl, pool, idx, num_accepted_tokens=acc)
    ref_idx = idx.clone()
    ref_idx[0, 1:] = -1
    ref_idx[2] = -1
    ref_pool = before.clone()
    o_ref = _decode(dev, wl, ref_pool, ref_idx, num_accepted_tokens=acc)
    for n in (0, 1):
        rows = _rows(o, wl, n)
        assert not torch.isnan(rows.float()).any(), n
        assert torch.equal(rows, _rows(o_ref, wl, n)), n
    assert (_rows(o, wl, 2) == 7.0).all()
    assert torch.equal(pool, ref_pool)
    assert not torch.equal(pool[5], before[5])                       # row 1's last token


def test_indexed_shared_slot_large_pool(rocm_device):
    """A pool of more than 4096 slots takes the per-tile form of the check (the workgroup
    scans the table at every tile): the same outcome."""
    dev = rocm_device
    N, nslots = 5, 5000
    wl = W.make(N, 1, 2, 4, 64, 64, seed=76, h0_scale=0.01)
    pool = 0.01 * torch.randn((nslots, 4, 64, 64), device=dev)
    before = pool.clone()
    idx = torch.tensor([4999, 17, 4200, 17, 3], dtype=torch.int32)   # 1 and 3 share 17
    o = _decode(dev, wl, pool, idx)
    ref_pool = before.clone()
    o_ref = _decode(dev, wl, ref_pool, torch.tensor([4999, -1, 4200, -1, 3], dtype=torch.int32))
    for n in (1, 3):
        assert torch.isnan(o[n].float()).all(), n
    for n in (0, 2, 4):
        assert torch.equal(o[n], o_ref[n]), n
    assert torch.equal(pool, ref_pool)
    assert not torch.equal(pool[4999], before[4999])
