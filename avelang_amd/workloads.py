"""Seeded synthetic workloads of the GDN hot path (the BASELINE configs).

Inputs (numpy PCG64, generated on the host then copied to the device):
    q, k ~ N(0,1), L2-normalised over K in fp32, then rounded to bf16
    v    ~ N(0,1), bf16
    beta = sigmoid(N(0,1)), fp32
    g    = -decay * softplus(N(0,1)), fp32   (decay 0.1; 0.01 for long context)
    h0   = h0_scale * N(0,1), fp32           (0 = no initial state)
The numpy view (``Workload.numpy()``) holds exactly the values the device
sees (bf16 values upcast to fp32), so a CPU checker consumes the same input.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

CONFIGS = {
    # name: (B, T, Hqk, Hv, K, V, decay, h0_scale)
    "cfg0_cpu_reference": dict(B=1, T=256, Hqk=4, Hv=4, K=64, V=64, decay=0.1, h0_scale=0.0),
    "cfg1_prefill_qwen3next": dict(B=1, T=8192, Hqk=16, Hv=32, K=128, V=128, decay=0.1, h0_scale=0.01),
    "cfg2_decode_b256": dict(B=256, T=1, Hqk=16, Hv=32, K=128, V=128, decay=0.1, h0_scale=0.01),
    "cfg3_varlen_64seq": dict(B=1, T=None, Hqk=16, Hv=32, K=128, V=128, decay=0.1, h0_scale=0.01,
                              nseq=64, len_lo=128, len_hi=4096),
    "cfg4_long_context": dict(B=1, T=65536, Hqk=16, Hv=32, K=128, V=128, decay=0.01, h0_scale=0.01),
}


def _softplus(x):
    return np.logaddexp(0.0, x)


def _bf16_round(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.float().numpy()


def varlen_cu_seqlens(nseq: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """cu_seqlens for ``nseq`` lengths uniform in [lo, hi] (inclusive), seeded."""
    rng = np.random.Generator(np.random.PCG64(seed + 7919))
    lens = rng.integers(lo, hi + 1, size=nseq)
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)


@dataclass
class Workload:
    q: np.ndarray          # fp32 holding bf16 values
    k: np.ndarray
    v: np.ndarray
    g: np.ndarray
    beta: np.ndarray
    h0: Optional[np.ndarray]
    cu_seqlens: Optional[np.ndarray]
    dims: dict = field(default_factory=dict)

    def numpy(self):
        return dict(q=self.q, k=self.k, v=self.v, g=self.g, beta=self.beta,
                    initial_state=self.h0, cu_seqlens=self.cu_seqlens)

    def torch(self, device="cuda"):
        bf = lambda x: torch.from_numpy(x).to(device=device, dtype=torch.bfloat16)  # noqa: E731
        f32 = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device)  # noqa: E731
        return dict(
            q=bf(self.q), k=bf(self.k), v=bf(self.v), g=f32(self.g), beta=f32(self.beta),
            initial_state=f32(self.h0),
            cu_seqlens=None if self.cu_seqlens is None else torch.from_numpy(self.cu_seqlens).to(device),
        )


def make(B: int, T: int, Hqk: int, Hv: int, K: int, V: int, seed: int = 0,
         decay: float = 0.1, h0_scale: float = 0.01, cu_seqlens=None,
         l2norm: bool = True) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((B, T, Hqk, K), dtype=np.float32)
    k = rng.standard_normal((B, T, Hqk, K), dtype=np.float32)
    if l2norm:
        q /= np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        k /= np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    v = rng.standard_normal((B, T, Hv, V), dtype=np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, Hv), dtype=np.float32)))).astype(np.float32)
    g = (-decay * _softplus(rng.standard_normal((B, T, Hv), dtype=np.float32))).astype(np.float32)
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    h0 = None
    if h0_scale:
        h0 = (h0_scale * rng.standard_normal((N, Hv, K, V), dtype=np.float32)).astype(np.float32)
    cu = None if cu_seqlens is None else np.asarray(cu_seqlens, dtype=np.int32)
    return Workload(_bf16_round(q), _bf16_round(k), _bf16_round(v), g, beta, h0, cu,
                    dims=dict(B=B, T=T, Hqk=Hqk, Hv=Hv, K=K, V=V, N=N))


def config(name: str, seed: int = 0, **override) -> Workload:
    c = dict(CONFIGS[name])
    c.update(override)
    cu = None
    if "nseq" in c:
        cu = varlen_cu_seqlens(c.pop("nseq"), c.pop("len_lo"), c.pop("len_hi"), seed)
        c["T"] = int(cu[-1])
    return make(seed=seed, cu_seqlens=cu, **c)
