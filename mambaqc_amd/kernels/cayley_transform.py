"""Cayley discretisation q = (1 - z/2)^-1 (x) (1 + z/2) on the GPU.

Mirrors mambaqc/kernels/cayley_transform.py:132-195. The HIP kernel uses the
closed form  q = (1 - |z|^2/4, v) / max(|1 - z/2|^2, eps)  for z = (a, v),
which equals the reference's inverse-then-product up to rounding.
"""
from __future__ import annotations

import torch

from .. import _native as nat


def cayley_discretization_fused(z: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """z: [batch, seq_len, d_model, d_state, 4] -> q of the same shape and dtype.

    Reference asserts: cayley_transform.py:151-152.
    """
    assert z.shape[-1] == 4, f"Last dim must be 4, got {z.shape[-1]}"
    assert z.ndim == 5, f"Expected 5D tensor, got {z.ndim}D"
    nat.require_device("cayley_discretization_fused", z)
    z = nat.aligned16(z)
    q = torch.empty_like(z)
    nat.call("mqc_cayley_fwd", z, z.data_ptr(), q.data_ptr(), z.numel() // 4, float(eps),
             nat.dtype_code(z), nat.stream_of(z))
    return q
