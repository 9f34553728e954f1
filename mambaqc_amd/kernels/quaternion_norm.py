"""Quaternion LayerNorm on the GPU.

Mirrors mambaqc/kernels/quaternion_norm.py:119-215 with the semantics of the
reference formula quaternion_layer_norm_reference (:219-245):
    n = sqrt(|q|^2 + eps); mu, var = mean, biased variance of n over d_model
    out = gamma * (n - mu) / sqrt(var + eps) * q / (n + eps) + beta
Statistics are exact over d_model for any width (the reference Triton kernel
pads the row to a power of two and lets the padding enter the statistics).
"""
from __future__ import annotations

import torch

from .. import _native as nat


def quaternion_layer_norm_fused(q: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor,
                                eps: float = 1e-5, return_stats: bool = False):
    """q: [batch, seq_len, d_model, 4]; gamma: [d_model]; beta: [d_model, 4].

    Reference asserts: quaternion_norm.py:142-145. With return_stats the
    per-row mean and 1/sqrt(var + eps) (fp32, [batch, seq_len]) are returned too.
    """
    assert q.shape[-1] == 4
    assert q.ndim == 4, f"Expected [B, T, D, 4], got {q.shape}"
    assert gamma.shape == (q.shape[2],), f"gamma shape mismatch: {gamma.shape}"
    assert beta.shape == (q.shape[2], 4), f"beta shape mismatch: {beta.shape}"
    nat.require_device("quaternion_layer_norm_fused", q, gamma, beta)
    B, T, D, _ = q.shape
    q = nat.aligned16(q)
    g = nat.aligned16(gamma.detach().float())
    b = nat.aligned16(beta.detach().float())
    out = torch.empty_like(q)
    mean = rstd = None
    if return_stats:
        mean = torch.empty(B, T, device=q.device, dtype=torch.float32)
        rstd = torch.empty(B, T, device=q.device, dtype=torch.float32)
    nat.call("mqc_qln_fwd", q, q.data_ptr(), g.data_ptr(), b.data_ptr(), out.data_ptr(),
             nat.ptr(mean), nat.ptr(rstd), B * T, D, float(eps), nat.dtype_code(q),
             nat.stream_of(q))
    return (out, mean, rstd) if return_stats else out


class QuaternionLayerNorm(torch.nn.Module):
    """Learnable quaternion layer normalisation (normalises norms, keeps directions).

    Same parameters as the reference (quaternion_norm.py:177-215): gamma [d_model]
    initialised to ones, beta [d_model, 4] initialised to zeros.
    """

    def __init__(self, d_model: int, eps: float = 1e-5):
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.gamma = torch.nn.Parameter(torch.ones(d_model))
        self.beta = torch.nn.Parameter(torch.zeros(d_model, 4))

    def forward(self, q: torch.Tensor) -> torch.Tensor:
        return quaternion_layer_norm_fused(q, self.gamma, self.beta, self.eps)

    def extra_repr(self) -> str:
        return f"d_model={self.d_model}, eps={self.eps}"
