"""chunk_gated_delta_rule's per-call save_for_backward, on the CPU: the
autograd forward allocates the backward's workspace (and hands it to the
forward call) exactly when the call or, with no per-call value, the module
default asks for it.  The library call itself is replaced by a recorder, so
no kernel runs."""
import pytest
import torch

from avelang_amd import gated_delta_rule as GDR


@pytest.mark.parametrize("default,per_call,expect", [
    (True, None, True), (False, None, False), (True, False, False), (False, True, True)])
def test_save_for_backward_per_call(monkeypatch, default, per_call, expect):
    seen = {}

    def fake_fwd(q, k, v, g, beta, scale, h0, oft, cu, l2, save_workspace=None, **kw):
        seen["ws"] = save_workspace
        B, T, Hqk, K = q.shape
        o = torch.zeros(v.shape, dtype=torch.bfloat16)
        return o, None

    monkeypatch.setattr(GDR, "_chunk_fwd", fake_fwd)
    monkeypatch.setattr(GDR, "SAVE_FORWARD_FOR_BACKWARD", default)
    B, T, Hqk, Hv, K, V = 1, 70, 2, 4, 64, 64
    q = torch.zeros(B, T, Hqk, K, dtype=torch.bfloat16, requires_grad=True)
    k = torch.zeros(B, T, Hqk, K, dtype=torch.bfloat16)
    v = torch.zeros(B, T, Hv, V, dtype=torch.bfloat16)
    g = torch.zeros(B, T, Hv)
    beta = torch.zeros(B, T, Hv)
    kw = {} if per_call is None else {"save_for_backward": per_call}
    GDR.chunk_gated_delta_rule(q, k, v, g, beta, **kw)
    ws = seen["ws"]
    if expect:
        need = GDR.chunk_bwd_workspace_bytes(B, T, Hqk, Hv, K, V, B, False, False)
        assert ws is not None and ws.dtype == torch.uint8 and ws.numel() >= need
    else:
        assert ws is None
