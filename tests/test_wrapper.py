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


# ------------------------------------------------------- layer operators ----
def test_layer_ops_validate_before_launch():
    from avelang_amd import layer_ops as L
    x = torch.zeros(2, 16, 8)
    w = torch.zeros(16, 4)
    with pytest.raises(ValueError, match="3-D"):
        L.causal_conv1d_fn(torch.zeros(16, 8), w)
    with pytest.raises(ValueError, match="kernel width"):
        L.causal_conv1d_fn(x, torch.zeros(16, 5))
    with pytest.raises(ValueError, match="activation"):
        L.causal_conv1d_fn(x, w, activation="relu")
    with pytest.raises(ValueError, match="ROCm"):
        L.causal_conv1d_fn(x, w, activation="silu")
    with pytest.raises(ValueError, match="conv_state length"):
        L.causal_conv1d_update(torch.zeros(2, 16), torch.zeros(2, 16, 2), w)
    with pytest.raises(ValueError, match="1 <= L <= 64"):
        L.causal_conv1d_update(torch.zeros(2, 16, 65), torch.zeros(2, 16, 3), w)
    with pytest.raises(ValueError, match="same shape"):
        L.fused_gdn_gating(torch.zeros(4), torch.zeros(3, 4), torch.zeros(3, 5), torch.zeros(4))
    with pytest.raises(ValueError, match="shape"):
        L.fused_gdn_gating(torch.zeros(3), torch.zeros(3, 4), torch.zeros(3, 4), torch.zeros(4))
    with pytest.raises(ValueError, match="64, 128 or 256"):
        L.l2norm_fwd(torch.zeros(3, 100))
    with pytest.raises(ValueError, match="match"):
        L.rms_norm_gated(torch.zeros(3, 128), torch.zeros(3, 64), torch.zeros(128))
    with pytest.raises(ValueError, match="float32, bfloat16 or float16"):
        L.rms_norm_gated(torch.zeros(3, 128, dtype=torch.float64),
                         torch.zeros(3, 128, dtype=torch.float64), torch.zeros(128))


def test_state_pool_validation():
    q, k, v, g, beta = _t(B=2, T=1)
    with pytest.raises(ValueError, match="state pool"):
        fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None,
                                         ssm_state_indices=torch.zeros(2, dtype=torch.int32))
    with pytest.raises(ValueError, match="in place"):
        fused_recurrent_gated_delta_rule(q, k, v, g, beta,
                                         initial_state=torch.zeros(3, 4, 128, 128),
                                         output_final_state=True, inplace_final_state=False,
                                         ssm_state_indices=torch.zeros(2, dtype=torch.int32))


def test_host_slot_table_rejects_shared_slots():
    from avelang_amd.gated_delta_rule import _check_distinct_slots
    _check_distinct_slots(torch.tensor([0, 2, -1, -1, 5], dtype=torch.int32), 6, "op")
    _check_distinct_slots(torch.tensor([[0, 1], [2, 9]], dtype=torch.int32), 6, "op")
    # a row may repeat its own slot (speculative decoding: several tokens' states into one)
    _check_distinct_slots(torch.tensor([[1, 1], [2, 3]], dtype=torch.int32), 6, "op")
    _check_distinct_slots(torch.zeros((0,), dtype=torch.int32), 6, "op")
    with pytest.raises(ValueError, match="two sequences the same slot"):
        _check_distinct_slots(torch.tensor([0, 2, 2], dtype=torch.int32), 6, "op")
    with pytest.raises(ValueError, match="two sequences the same slot"):
        _check_distinct_slots(torch.tensor([[0, 1], [1, 3]], dtype=torch.int32), 6, "op")
