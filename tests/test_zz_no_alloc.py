"""gdn_chunk_fwd_noalloc: the chunked prefill on the library's own device
scratch, called through the C ABI, against gdn_chunk_fwd with a caller
workspace on the same inputs (the same kernels: bit-exact).  Two calls in a
row, the second smaller, so the second runs on scratch the first left
behind; and a problem over the scratch limit is rejected before launch.
"""
import numpy as np
import pytest
import torch

from avelang_amd import _native
from avelang_amd import workloads as W

pytestmark = pytest.mark.gpu


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _run(lib, dev, wl, noalloc):
    t = wl.torch(dev)
    B, T, Hqk, K = t["q"].shape
    Hv, V = t["v"].shape[2], t["v"].shape[3]
    cu = t["cu_seqlens"]
    N = B if cu is None else cu.numel() - 1
    o = torch.full_like(t["v"], 5.0)
    ht = torch.full((N, Hv, K, V), 5.0, dtype=torch.float32, device=dev)
    args = [t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), t["g"].data_ptr(),
            t["beta"].data_ptr(), t["initial_state"].data_ptr(), ht.data_ptr(), o.data_ptr(),
            None if cu is None else cu.data_ptr(), B, T, Hqk, Hv, K, V, N, K ** -0.5, 0]
    if noalloc:
        rc = lib.gdn_chunk_fwd_noalloc(*args, _stream(dev))
    else:
        nbytes = lib.gdn_chunk_workspace_bytes(B, T, Hqk, Hv, K, V, N, int(cu is not None), 0)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        rc = lib.gdn_chunk_fwd(*args, ws.data_ptr(), nbytes, _stream(dev))
    assert rc == 0, lib.gdn_last_error().decode()
    torch.cuda.synchronize()
    return o, ht


def test_noalloc_matches_workspace_form_twice(rocm_device):
    lib = _native.lib()
    big = W.make(1, 1000, 16, 32, 128, 128, seed=71, h0_scale=0.01,
                 cu_seqlens=np.array([0, 300, 301, 1000], dtype=np.int32))
    small = W.make(2, 200, 4, 8, 128, 128, seed=72, h0_scale=0.01)
    for what, wl in (("first call", big), ("second, smaller call", small)):
        o_ref, s_ref = _run(lib, rocm_device, wl, noalloc=False)
        o, s = _run(lib, rocm_device, wl, noalloc=True)
        assert torch.equal(o, o_ref), f"{what}: o differs"
        assert torch.equal(s, s_ref), f"{what}: final state differs"
        assert o.abs().sum() > 0


def test_noalloc_rejects_problems_over_the_scratch_limit(rocm_device):
    lib = _native.lib()
    # config 1 (T = 8192, 32 v-heads) needs far more than 32 MiB of scratch
    need = lib.gdn_chunk_workspace_bytes(1, 8192, 16, 32, 128, 128, 1, 0, 0)
    assert need > (32 << 20)
    fake = [1 << 28, 2 << 28, 3 << 28, 4 << 28, 5 << 28, None, None, 6 << 28, None]
    rc = lib.gdn_chunk_fwd_noalloc(*fake, 1, 8192, 16, 32, 128, 128, 1, 0.1, 0, None)
    assert rc == -4 and "scratch" in lib.gdn_last_error().decode()
