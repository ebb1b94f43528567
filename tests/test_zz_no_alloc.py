"""gdn_chunk_fwd_noalloc: the chunked prefill on the library's own device
scratch, called through the C ABI, against gdn_chunk_fwd with a caller
workspace on the same inputs (the same kernels: bit-exact).  Two calls in a
row, the second smaller, so the second runs on scratch the first left
behind; a problem just over the scratch limit is rejected before anything
is enqueued (real device tensors, so a regression of that check would run
rather than touch memory it does not own); and the entry point captured in
a HIP graph replays bit-exactly, also when its very first call in the
process is made under capture (a fresh process).
"""
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from avelang_amd import _native
from avelang_amd import workloads as W

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _limit():
    text = open(os.path.join(ROOT, "include", "gdn.h")).read()
    m = re.search(r"#define GDN_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    return int(m.group(1)) << int(m.group(2))


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _args(t, o, ht, K):
    B, T, Hqk, _ = t["q"].shape
    Hv, V = t["v"].shape[2], t["v"].shape[3]
    cu = t["cu_seqlens"]
    N = B if cu is None else cu.numel() - 1
    return [t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), t["g"].data_ptr(),
            t["beta"].data_ptr(), t["initial_state"].data_ptr(), ht.data_ptr(), o.data_ptr(),
            None if cu is None else cu.data_ptr(), B, T, Hqk, Hv, K, V, N, K ** -0.5, 0]


def _outputs(t, dev):
    B, T, Hqk, K = t["q"].shape
    Hv, V = t["v"].shape[2], t["v"].shape[3]
    cu = t["cu_seqlens"]
    N = B if cu is None else cu.numel() - 1
    return torch.full_like(t["v"], 5.0), torch.full((N, Hv, K, V), 5.0, dtype=torch.float32,
                                                     device=dev)


def _run(lib, dev, wl, noalloc):
    t = wl.torch(dev)
    K = t["q"].shape[3]
    o, ht = _outputs(t, dev)
    args = _args(t, o, ht, K)
    if noalloc:
        rc = lib.gdn_chunk_fwd_noalloc(*args, _stream(dev))
    else:
        B, T, Hqk, _ = t["q"].shape
        Hv, V = t["v"].shape[2], t["v"].shape[3]
        cu = t["cu_seqlens"]
        nbytes = lib.gdn_chunk_workspace_bytes(B, T, Hqk, Hv, K, V, args[15],
                                               int(cu is not None), 0)
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
    """The smallest T (at 16 -> 32 heads, K = V = 128) whose workspace exceeds the scratch:
    real tensors of that shape, the call returns GDN_ERR_WORKSPACE and o keeps its fill."""
    lib = _native.lib()
    limit = _limit()
    T = 64
    while lib.gdn_chunk_workspace_bytes(1, T, 16, 32, 128, 128, 1, 0, 0) <= limit:
        T += 64
    assert lib.gdn_chunk_workspace_bytes(1, T - 64, 16, 32, 128, 128, 1, 0, 0) <= limit
    wl = W.make(1, T, 16, 32, 128, 128, seed=73, h0_scale=0.01)
    t = wl.torch(rocm_device)
    o, ht = _outputs(t, rocm_device)
    rc = lib.gdn_chunk_fwd_noalloc(*_args(t, o, ht, 128), _stream(rocm_device))
    torch.cuda.synchronize()
    assert rc == -4 and "scratch" in lib.gdn_last_error().decode()
    assert bool((o == 5.0).all()) and bool((ht == 5.0).all())


def _captured_replays(lib, dev, wl, warm):
    """o, ht of three replays of a graph holding one noalloc call (eager work and a
    synchronisation between replays), and of the eager workspace form."""
    o_ref, s_ref = _run(lib, dev, wl, noalloc=False)
    t = wl.torch(dev)
    o, ht = _outputs(t, dev)
    args = _args(t, o, ht, t["q"].shape[3])
    if warm:
        assert lib.gdn_chunk_fwd_noalloc(*args, _stream(dev)) == 0
        torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.gdn_chunk_fwd_noalloc(*args, side.cuda_stream)
    assert rc == 0, lib.gdn_last_error().decode()
    out = []
    for i in range(3):
        o.fill_(float(i + 7))
        ht.fill_(float(i + 7))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        out.append((o.clone(), ht.clone()))
    return out, (o_ref, s_ref)


def test_noalloc_graph_capture_replays(rocm_device):
    lib = _native.lib()
    wl = W.make(1, 300, 4, 8, 128, 128, seed=74, h0_scale=0.01)
    reps, (o_ref, s_ref) = _captured_replays(lib, rocm_device, wl, warm=True)
    for i, (o, s) in enumerate(reps):
        assert torch.equal(o, o_ref), f"replay {i}: o differs"
        assert torch.equal(s, s_ref), f"replay {i}: final state differs"


_FRESH = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[2])
from avelang_amd import _native
from avelang_amd import workloads as W
import test_zz_no_alloc as M
lib = _native.lib()
dev = torch.device("cuda:0")
wl = W.make(1, 300, 4, 8, 128, 128, seed=75, h0_scale=0.01)
reps, (o_ref, s_ref) = M._captured_replays(lib, dev, wl, warm=False)
ok = all(torch.equal(o, o_ref) and torch.equal(s, s_ref) for o, s in reps)
print("FRESH_OK" if ok else "FRESH_MISMATCH", flush=True)
"""


def test_noalloc_first_call_under_capture(rocm_device):
    """In a fresh process the very first gdn_chunk_fwd_noalloc call (which looks the scratch
    address up) is made under stream capture; its replays equal the workspace form."""
    torch.cuda.synchronize()
    r = subprocess.run([sys.executable, "-c", _FRESH, ROOT, os.path.join(ROOT, "tests")],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "FRESH_OK" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
