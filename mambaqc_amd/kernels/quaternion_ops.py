"""Quaternion element-wise operators on the GPU.

Mirrors mambaqc/kernels/quaternion_ops.py (the reference's operator API):
same names, argument meaning and shape assertions; each call runs one HIP
kernel of libmambaqc_hip.so on the tensor's device and current stream and
returns a new tensor. There is no CPU path: CPU tensors raise RuntimeError.
"""
from __future__ import annotations

import torch

from .. import _native as nat


def _same_dtype(name: str, *ts: torch.Tensor) -> None:
    for t in ts[1:]:
        if t.dtype != ts[0].dtype:
            raise TypeError(f"{name}: dtype mismatch {ts[0].dtype} vs {t.dtype}")


def quaternion_multiply(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """Hamilton product p (x) q of [..., 4] tensors of equal shape.

    Reference: quaternion_ops.py:259-303 (shape asserts :270-271).
    """
    assert p.shape == q.shape, f"Shape mismatch: {p.shape} vs {q.shape}"
    assert p.shape[-1] == 4, f"Last dim must be 4, got {p.shape[-1]}"
    nat.require_device("quaternion_multiply", p, q)
    _same_dtype("quaternion_multiply", p, q)
    p = nat.aligned16(p)
    q = nat.aligned16(q)
    out = torch.empty_like(p, memory_format=torch.contiguous_format)
    n = p.numel() // 4
    nat.call("mqc_quaternion_multiply", p, p.data_ptr(), q.data_ptr(), out.data_ptr(), n,
             nat.dtype_code(p), nat.stream_of(p))
    return out


def quaternion_multiply_batched(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """Hamilton product of [B, T, D, S, 4] tensors. Reference: quaternion_ops.py:306-357."""
    assert p.shape == q.shape
    assert p.shape[-1] == 4
    assert p.ndim == 5, f"Expected 5D tensor, got {p.ndim}D"
    return quaternion_multiply(p, q)


def quaternion_conjugate(q: torch.Tensor) -> torch.Tensor:
    """(w, -x, -y, -z). Reference: quaternion_ops.py:360-391."""
    assert q.shape[-1] == 4
    nat.require_device("quaternion_conjugate", q)
    q = nat.aligned16(q)
    out = torch.empty_like(q)
    nat.call("mqc_quaternion_conjugate", q, q.data_ptr(), out.data_ptr(), q.numel() // 4,
             nat.dtype_code(q), nat.stream_of(q))
    return out


def quaternion_inverse(q: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """conj(q) / max(|q|^2, eps). Reference: quaternion_ops.py:394-428 (clamp :409)."""
    assert q.shape[-1] == 4
    nat.require_device("quaternion_inverse", q)
    q = nat.aligned16(q)
    out = torch.empty_like(q)
    nat.call("mqc_quaternion_inverse", q, q.data_ptr(), out.data_ptr(), q.numel() // 4,
             float(eps), nat.dtype_code(q), nat.stream_of(q))
    return out


def quaternion_norm(q: torch.Tensor) -> torch.Tensor:
    """|q| over the last axis, shape q.shape[:-1]. Reference: quaternion_ops.py:431-461."""
    assert q.shape[-1] == 4
    nat.require_device("quaternion_norm", q)
    q = nat.aligned16(q)
    out = torch.empty(q.shape[:-1], dtype=q.dtype, device=q.device)
    nat.call("mqc_quaternion_norm", q, q.data_ptr(), out.data_ptr(), q.numel() // 4,
             nat.dtype_code(q), nat.stream_of(q))
    return out
