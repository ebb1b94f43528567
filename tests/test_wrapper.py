"""Host-side validation of the Python operators (no GPU needed): every
problem is rejected with ValueError before the native library is called,
mirroring python/avelang_kernels/amdgpu_gemm.py:463-486."""
import pytest
import torch

from avelang_amd import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule

OPS = [chunk_gated_delta_rule, fused_recurrent_gated_delta_rule]


def _t(B=1, T=8, Hqk=2, Hv=4, K=128, V=128, dtype=torch.bfloat16, device="cpu"):
    q = torch.zeros(B, T, Hqk, K, dtype=dtype, device=device)
    k = torch.zeros(B, T, Hqk, K, dtype=dtype, device=device)
    v = torch.zeros(B, T, Hv, V, dtype=dtype, device=device)
    g = torch.zeros(B, T, Hv, device=device)
    beta = torch.zeros(B, T, Hv, device=device)
    return q, k, v, g, beta


@pytest.mark.parametrize("op", OPS)
def test_requires_rocm_device(op):
    with pytest.raises(ValueError, match="ROCm"):
        op(*_t())


@pytest.mark.parametrize("op", OPS)
def test_requires_bf16(op):
    with pytest.raises(ValueError, match="bfloat16"):
        op(*_t(dtype=torch.float32))


@pytest.mark.parametrize("op", OPS)
def test_shape_checks(op):
    q, k, v, g, beta = _t()
    with pytest.raises(ValueError, match="k must have shape"):
        op(q, k[:, :4], v, g, beta)
    with pytest.raises(ValueError, match="multiple of qk-heads"):
        op(*_t(Hqk=3, Hv=4))
    with pytest.raises(ValueError, match="unsupported"):
        op(*_t(K=96))
    with pytest.raises(ValueError, match="g must have shape"):
        op(q, k, v, g[:, :, :2], beta)


@pytest.mark.parametrize("op", OPS)
def test_cu_seqlens_checks(op):
    q, k, v, g, beta = _t(B=2)
    with pytest.raises(ValueError, match="batch size 1"):
        op(q, k, v, g, beta, cu_seqlens=torch.tensor([0, 8], dtype=torch.int32))
    q, k, v, g, beta = _t()
    with pytest.raises(ValueError, match="int32 or int64"):
        op(q, k, v, g, beta, cu_seqlens=torch.tensor([0.0, 8.0]))
