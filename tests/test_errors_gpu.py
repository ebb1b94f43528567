"""A HIP error already pending on the calling thread (left by someone else's
failed call) is not reported as the library's own: the entry points clear it
before their launches, so a valid call returns 0 and leaves no error behind.
The pending error is made with a failing hipSetDevice on the HIP runtime the
process already loaded (the one libgdn.so is bound to)."""
import ctypes

import pytest
import torch

from avelang_amd import _native
from avelang_amd import workloads as W

pytestmark = pytest.mark.gpu


def _hip_runtime():
    for line in open("/proc/self/maps"):
        if "libamdhip64.so" in line:
            return ctypes.CDLL(line.split()[-1])
    pytest.fail("libamdhip64.so is not mapped in this process")


@pytest.mark.parametrize("entry", ["chunk", "recurrent"])
def test_foreign_pending_error_is_not_reported(rocm_device, entry):
    from avelang_amd import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
    hip = _hip_runtime()
    wl = W.make(1, 100, 2, 4, 128, 128, seed=81, h0_scale=0.01)
    t = wl.torch(rocm_device)
    torch.cuda.synchronize()
    assert hip.hipSetDevice(9999) != 0          # leaves hipErrorInvalidDevice pending
    assert hip.hipPeekAtLastError() != 0
    fn = chunk_gated_delta_rule if entry == "chunk" else fused_recurrent_gated_delta_rule
    o, s = fn(t["q"], t["k"], t["v"], t["g"], t["beta"], initial_state=t["initial_state"],
              output_final_state=True)          # raises if the call reports an error
    torch.cuda.synchronize()
    assert hip.hipGetLastError() == 0
    assert torch.isfinite(o.float()).all() and s.abs().sum() > 0
    assert _native.lib() is not None
