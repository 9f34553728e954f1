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


def _qln_forward(q, gamma, beta, eps, want_stats):
    B, T, D, _ = q.shape
    q = nat.aligned16(q.detach())
    g = nat.param_f32(gamma)
    b = nat.param_f32(beta)
    out = torch.empty_like(q)
    mean = rstd = None
    if want_stats:
        mean = torch.empty(B, T, device=q.device, dtype=torch.float32)
        rstd = torch.empty(B, T, device=q.device, dtype=torch.float32)
    nat.call("mqc_qln_fwd", q, q.data_ptr(), g.data_ptr(), b.data_ptr(), out.data_ptr(),
             nat.ptr(mean), nat.ptr(rstd), B * T, D, float(eps), nat.dtype_code(q),
             nat.stream_of(q))
    return out, mean, rstd, q, g


class _QLNFunction(torch.autograd.Function):
    """Autograd wrapper: HIP forward (saving mean and rstd) and HIP backward."""

    @staticmethod
    def forward(ctx, q, gamma, beta, eps):
        out, mean, rstd, qc, g = _qln_forward(q, gamma, beta, eps, True)
        ctx.save_for_backward(qc, g, mean, rstd)
        ctx.meta = (eps, gamma.dtype, beta.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        qc, g, mean, rstd = ctx.saved_tensors
        eps, t_gamma, t_beta = ctx.meta
        dq, dgamma, dbeta = _qln_backward(qc, g, mean, rstd, dout, eps)
        return dq, dgamma.to(t_gamma), dbeta.to(t_beta), None


def _qln_backward(qc, g, mean, rstd, dout, eps):
    """(dq in q's dtype, dgamma [D] and dbeta [D, 4] in fp32) from the forward's
    operands (q in the kernel's form, gamma fp32) and statistics."""
    B, T, D, _ = qc.shape
    dout = nat.aligned16(dout.to(qc.dtype))
    dq = torch.empty_like(qc)
    ne = torch.empty(B * T, D, device=qc.device, dtype=torch.float32)
    nat.call("mqc_qln_bwd", qc, qc.data_ptr(), dout.data_ptr(), g.data_ptr(),
             mean.data_ptr(), rstd.data_ptr(), dq.data_ptr(), ne.data_ptr(), B * T, D,
             float(eps), nat.dtype_code(qc), nat.stream_of(qc))
    return dq, ne.sum(0), dout.float().reshape(B * T, D, 4).sum(0)


def quaternion_layer_norm_fused(q: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor,
                                eps: float = 1e-5, return_stats: bool = False):
    """q: [batch, seq_len, d_model, 4]; gamma: [d_model]; beta: [d_model, 4].

    Reference asserts: quaternion_norm.py:142-145. With return_stats the
    per-row mean and 1/sqrt(var + eps) (fp32, [batch, seq_len]) are returned too.
    Differentiable in q, gamma and beta when autograd is recording.
    """
    assert q.shape[-1] == 4
    assert q.ndim == 4, f"Expected [B, T, D, 4], got {q.shape}"
    assert gamma.shape == (q.shape[2],), f"gamma shape mismatch: {gamma.shape}"
    assert beta.shape == (q.shape[2], 4), f"beta shape mismatch: {beta.shape}"
    if nat.compiling():
        out, mean, rstd = torch.ops.mambaqc.quaternion_layer_norm(q, gamma, beta, eps)
        return (out, mean, rstd) if return_stats else out
    nat.require_device("quaternion_layer_norm_fused", q, gamma, beta)
    if (torch.is_grad_enabled() and not return_stats
            and any(t.requires_grad for t in (q, gamma, beta))):
        return _QLNFunction.apply(q, gamma, beta, eps)
    out, mean, rstd, _, _ = _qln_forward(q, gamma, beta, eps, return_stats)
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
