"""Cumulative left-ordered Hamilton product along the sequence axis.

Mirrors parallel_scan_quaternion, mambaqc/kernels/parallel_scan.py:171-264,
with the semantics of its sequential reference (:267-295):
    cumulative[:, t] = q[:, t] (x) q[:, t-1] (x) ... (x) q[:, 0]
The HIP kernel scans the true time axis for every (b, d, k) lane; it does not
reproduce the reference GPU path's reshape of a [B,T,D,S,4] tensor to
[B*D, T, S, 4], which mixes the time and d_model axes whenever D > 1.
"""
from __future__ import annotations

import torch

from .. import _native as nat


def parallel_scan_quaternion(q_sequence: torch.Tensor) -> torch.Tensor:
    """q_sequence: [batch, seq_len, d_model, d_state, 4] -> cumulative products (new tensor)."""
    assert q_sequence.shape[-1] == 4
    assert q_sequence.ndim == 5
    nat.require_device("parallel_scan_quaternion", q_sequence)
    q = nat.aligned16(q_sequence)
    B, T, D, S, _ = q.shape
    out = torch.empty_like(q)
    nat.call("mqc_cumprod_scan_fwd", q, q.data_ptr(), out.data_ptr(), B, T, D * S,
             nat.dtype_code(q), nat.stream_of(q))
    return out
