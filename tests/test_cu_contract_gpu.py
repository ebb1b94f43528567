"""Device-side cu_seqlens contract of the chunked entry points.

cu_seqlens on the device is not read on the host.  The chunk table kernel
checks cu[0] == 0, non-decreasing, cu[N] == T; on a violation every sequence
is treated as empty: o and the gradients are zero-filled, the final state
equals the initial state and dh0 equals dht (include/gdn.h).  The outputs are
pre-filled with non-zero values so that a missing write cannot pass.
"""
import numpy as np
import pytest
import torch

from avelang_amd import workloads as W

pytestmark = pytest.mark.gpu

BAD = {
    "decreasing": [0, 100, 50, 230],
    "short_total": [0, 70, 200],
    "nonzero_start": [5, 70, 230],
    "overshoot": [0, 70, 300],
}


def _workload(dev, cu):
    wl = W.make(1, 230, 2, 4, 128, 128, seed=60, h0_scale=0.01,
                cu_seqlens=np.array([0, 70, 230], dtype=np.int32))
    t = wl.torch(dev)
    t["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32, device=dev)
    return t


@pytest.mark.parametrize("case", sorted(BAD))
def test_forward_violation_empties_every_sequence(rocm_device, case):
    from avelang_amd import chunk_gated_delta_rule
    t = _workload(rocm_device, BAD[case])
    N = len(BAD[case]) - 1
    h0 = torch.randn((N, 4, 128, 128), device=rocm_device) * 0.01
    out = torch.full_like(t["v"], 7.0)
    o, ht = chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                   initial_state=h0, output_final_state=True,
                                   cu_seqlens=t["cu_seqlens"], out=out)
    torch.cuda.synchronize()
    assert o.data_ptr() == out.data_ptr()
    assert not o.any(), f"{case}: o not zero-filled"
    assert torch.equal(ht, h0), f"{case}: final state != initial state"


@pytest.mark.parametrize("case", sorted(BAD))
def test_backward_violation_zero_gradients(rocm_device, case):
    from avelang_amd import chunk_gated_delta_rule_bwd
    t = _workload(rocm_device, BAD[case])
    N = len(BAD[case]) - 1
    h0 = torch.randn((N, 4, 128, 128), device=rocm_device) * 0.01
    dht = torch.randn((N, 4, 128, 128), device=rocm_device) * 0.01
    do = torch.randn_like(t["v"], dtype=torch.float32).to(torch.bfloat16)
    # leave non-zero bytes in the blocks the gradients will be allocated from
    junk = [torch.full_like(t[n], 3.0) for n in ("q", "k", "v", "g", "beta")]
    del junk
    dq, dk, dv, dg, db, dh0 = chunk_gated_delta_rule_bwd(
        t["q"], t["k"], t["v"], t["g"], t["beta"], do, dht, initial_state=h0,
        cu_seqlens=t["cu_seqlens"])
    torch.cuda.synchronize()
    for name, x in (("dq", dq), ("dk", dk), ("dv", dv), ("dg", dg), ("dbeta", db)):
        assert not x.any(), f"{case}: {name} not zero-filled"
    assert torch.equal(dh0, dht), f"{case}: dh0 != dht"


def test_valid_device_cu_seqlens_unaffected(rocm_device):
    """A valid device cu_seqlens gives the same result as the host copy."""
    from avelang_amd import chunk_gated_delta_rule
    t = _workload(rocm_device, [0, 70, 230])
    o1, s1 = chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                    initial_state=t["initial_state"], output_final_state=True,
                                    cu_seqlens=t["cu_seqlens"])
    o2, s2 = chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                    initial_state=t["initial_state"], output_final_state=True,
                                    cu_seqlens=t["cu_seqlens"].cpu())
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    assert o1.abs().sum() > 0
