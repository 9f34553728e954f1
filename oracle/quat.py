"""Quaternion math of the reference's CPU path, restated in plain torch (CPU).

Test infrastructure only (see oracle/__init__.py). Citations are into
/root/reference/mambaqc (polux06/mambaqc).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

IDENTITY = (1.0, 0.0, 0.0, 0.0)


def _cpu(*ts):
    for t in ts:
        if t.is_cuda:
            raise RuntimeError("oracle functions take CPU tensors")


def hamilton(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """p (x) q over the last axis, broadcasting leading axes.

    kernels/quaternion_ops.py:273-282 (the torch fallback of quaternion_multiply).
    """
    _cpu(p, q)
    p0, p1, p2, p3 = p.unbind(-1)
    q0, q1, q2, q3 = q.unbind(-1)
    r0 = p0 * q0 - p1 * q1 - p2 * q2 - p3 * q3
    r1 = p0 * q1 + p1 * q0 + p2 * q3 - p3 * q2
    r2 = p0 * q2 - p1 * q3 + p2 * q0 + p3 * q1
    r3 = p0 * q3 + p1 * q2 - p2 * q1 + p3 * q0
    return torch.stack((r0, r1, r2, r3), dim=-1)


def conjugate(q: torch.Tensor) -> torch.Tensor:
    """kernels/quaternion_ops.py:372-374."""
    _cpu(q)
    return q * torch.tensor([1.0, -1.0, -1.0, -1.0], dtype=q.dtype)


def inverse(q: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """conj(q) / max(|q|^2, eps). kernels/quaternion_ops.py:407-410."""
    _cpu(q)
    norm_sq = (q * q).sum(dim=-1, keepdim=True).clamp_min(eps)
    return conjugate(q) / norm_sq


def norm(q: torch.Tensor) -> torch.Tensor:
    """kernels/quaternion_ops.py:443-444."""
    _cpu(q)
    return torch.linalg.vector_norm(q, dim=-1)


def cayley_reference(z: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """(1 - z/2)^-1 (x) (1 + z/2). kernels/cayley_transform.py:199-223."""
    _cpu(z)
    one = torch.zeros_like(z)
    one[..., 0] = 1.0
    numerator = one + 0.5 * z
    denominator = one - 0.5 * z
    return hamilton(inverse(denominator, eps=eps), numerator)


def cumprod_reference(q: torch.Tensor) -> torch.Tensor:
    """cum[:, t] = q[:, t] (x) cum[:, t-1], cum[:, -1] = 1 along axis 1.

    kernels/parallel_scan.py:267-295 (left multiplication, :290-293).
    """
    _cpu(q)
    out = torch.zeros_like(q)
    acc = torch.zeros_like(q[:, 0])
    acc[..., 0] = 1.0
    for t in range(q.shape[1]):
        acc = hamilton(q[:, t], acc)
        out[:, t] = acc
    return out


def ssm_step_reference(q, B, S, C, D, h_prev):
    """One step: h = q (x) h_prev + B (x) S; y = sum_k C (x) h + D * S.

    kernels/ssm_fused.py:405-430, with S broadcast over d_state (deviation D2).
    q, B, C, h_prev: [b, d, k, 4]; S: [b, d, 4]; D: [b, d].
    """
    _cpu(q, B, S, C, D, h_prev)
    h_new = hamilton(q, h_prev) + hamilton(B, S.unsqueeze(2))
    y = hamilton(C, h_new).sum(dim=2) + D.unsqueeze(-1) * S
    return h_new, y


def ssm_forward_reference(q, B, S, C, D, h0=None, return_state=False):
    """All steps from h0 (zeros by default). kernels/ssm_fused.py:363-379.

    q, B, C: [b, T, d, k, 4]; S: [b, T, d, 4]; D: [b, T, d] -> y [b, T, d, 4].
    """
    _cpu(q, B, S, C, D)
    b, T, d, k, _ = q.shape
    h = torch.zeros(b, d, k, 4, dtype=q.dtype) if h0 is None else h0.clone()
    y = torch.empty(b, T, d, 4, dtype=q.dtype)
    for t in range(T):
        h, y[:, t] = ssm_step_reference(q[:, t], B[:, t], S[:, t], C[:, t], D[:, t], h)
    return (y, h) if return_state else y


def lambda_from_params(lambda_alpha: torch.Tensor, lambda_imag: torch.Tensor) -> torch.Tensor:
    """Lambda = (-softplus(alpha), tanh(v)) as [d, k, 4].

    models/quaternion_mamba2_block.py:206-212.
    """
    _cpu(lambda_alpha, lambda_imag)
    lam = torch.zeros(*lambda_alpha.shape, 4, dtype=lambda_alpha.dtype)
    lam[..., 0] = -F.softplus(lambda_alpha)
    lam[..., 1:] = torch.tanh(lambda_imag)
    return lam


def ssm_forward_dl_reference(delta, s, B, C, lambda_alpha, lambda_imag, D, eps=1e-6,
                             h0=None, return_state=False):
    """The block's SSM given delta, the real signal s and the raw Lambda params.

    models/quaternion_mamba2_block.py:194-228: S = (s, 0, 0, 0) (:200-202),
    z = delta * Lambda (:217-221), q = Cayley(z, eps) (:224-225),
    y = ssm_forward(q, B, S, C, D expanded over (b, t)) (:194, :228).
    delta, s: [b, T, d]; B, C: [b, T, d, k, 4]; D: [d].
    """
    _cpu(delta, s, B, C, lambda_alpha, lambda_imag, D)
    b, T, d = delta.shape
    lam = lambda_from_params(lambda_alpha, lambda_imag)
    z = delta[..., None, None] * lam[None, None]
    q = cayley_reference(z, eps=eps)
    S = torch.zeros(b, T, d, 4, dtype=s.dtype)
    S[..., 0] = s
    Dx = D.unsqueeze(0).unsqueeze(0).expand(b, T, d)
    return ssm_forward_reference(q, B, S, C, Dx, h0=h0, return_state=return_state)


def qln_reference(q: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor,
                  eps: float = 1e-5) -> torch.Tensor:
    """Quaternion LayerNorm. kernels/quaternion_norm.py:219-245.

    q: [..., d, 4]; gamma: [d]; beta: [d, 4]. Statistics over the d axis.
    """
    _cpu(q, gamma, beta)
    n = torch.sqrt((q ** 2).sum(dim=-1) + eps)
    mean = n.mean(dim=-1, keepdim=True)
    var = n.var(dim=-1, keepdim=True, unbiased=False)
    n_hat = (n - mean) / torch.sqrt(var + eps)
    direction = q / (n.unsqueeze(-1) + eps)
    return gamma.unsqueeze(-1) * n_hat.unsqueeze(-1) * direction + beta
