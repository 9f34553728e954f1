"""Depthwise causal 1-D convolution (torch op; not a custom kernel).

Same module, parameters and initialisation as
mambaqc/layers/causal_conv1d.py:17-97: an nn.Conv1d with groups = channels
whose weight is re-drawn with xavier_uniform_ and whose bias is zeroed, applied
after k-1 zeros of left padding so output t sees inputs t-k+1 .. t.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _native as nat


class CausalConv1d(nn.Module):
    def __init__(self, d_model: int, kernel_size: int = 4, bias: bool = True):
        super().__init__()
        self.d_model = d_model
        self.kernel_size = kernel_size
        self.padding = kernel_size - 1
        self.conv = nn.Conv1d(d_model, d_model, kernel_size, padding=0, groups=d_model, bias=bias)
        nn.init.xavier_uniform_(self.conv.weight)
        if self.conv.bias is not None:
            nn.init.zeros_(self.conv.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: [batch, seq_len, channels] -> same shape."""
        xt = x.transpose(1, 2)
        if self.padding > 0:
            xt = F.pad(xt, (self.padding, 0))
        return self.conv(xt).transpose(1, 2)

    def extra_repr(self) -> str:
        return (f"d_model={self.d_model}, kernel_size={self.kernel_size}, "
                f"padding={self.padding}, bias={self.conv.bias is not None}")


CausalConv1D = CausalConv1d


def _rows_view(x: torch.Tensor):
    """(x, row stride) with x's rows uniformly strided and its last axis dense;
    otherwise a contiguous copy."""
    B, T, C = x.shape
    if x.stride(-1) != 1 or x.stride(0) != T * x.stride(1):
        x = x.contiguous()
    return x, x.stride(1)


class _ConvSiLU(torch.autograd.Function):
    """silu(causal depthwise conv1d(x)) with HIP forward and backward."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        B, T, C = x.shape
        K = weight.shape[-1]
        xv, xs = _rows_view(x.detach())
        w = nat.param_f32(weight).reshape(C, K)
        b = None if bias is None else nat.param_f32(bias)
        out = torch.empty(B, T, C, device=x.device, dtype=x.dtype)
        nat.call("mqc_causal_conv_silu_fwd", xv, xv.data_ptr(), xs, w.data_ptr(), nat.ptr(b),
                 out.data_ptr(), B, T, C, K, nat.dtype_code(xv), nat.stream_of(xv))
        ctx.save_for_backward(xv, w, b)
        ctx.meta = (xs, tuple(weight.shape), weight.dtype,
                    None if bias is None else bias.dtype)
        return out

    @staticmethod
    def backward(ctx, gout):
        xv, w, b = ctx.saved_tensors
        xs, wshape, t_w, t_b = ctx.meta
        dx, dw, db = _conv_silu_backward(xv, xs, w, b, gout)
        return (dx, dw.reshape(wshape).to(t_w), None if t_b is None else db.to(t_b))


def _conv_silu_backward(xv, xs, w, b, gout):
    """(dx [B, T, C] in x's dtype, dweight [C, K] and dbias [C] in fp32) from the
    forward's operands: x as a row view with row stride xs, weight [C, K] and
    bias (or None) in fp32."""
    B, T, C = xv.shape
    K = w.shape[1]
    gout = nat.aligned16(gout.to(xv.dtype))
    R = nat.load().mqc_conv_run_length()
    rows = B * ((T + R - 1) // R)
    dx = torch.empty(B, T, C, device=xv.device, dtype=xv.dtype)
    dw = torch.empty(rows, C, K, device=xv.device, dtype=torch.float32)
    db = torch.empty(rows, C, device=xv.device, dtype=torch.float32)
    nat.call("mqc_causal_conv_silu_bwd", xv, xv.data_ptr(), xs, w.data_ptr(), nat.ptr(b),
             gout.data_ptr(), dx.data_ptr(), C, dw.data_ptr(), db.data_ptr(), B, T, C, K,
             nat.dtype_code(xv), nat.stream_of(xv))
    return dx, dw.sum(0), db.sum(0)


def causal_conv1d_silu(x: torch.Tensor, weight: torch.Tensor,
                       bias: torch.Tensor | None) -> torch.Tensor:
    """silu(CausalConv1d(x)) in one HIP pass: x [batch, seq_len, channels] (may be
    the strided first half of in_proj's output), weight [channels, 1, k] (the
    Conv1d's), bias [channels] or None -> dense [batch, seq_len, channels].
    Differentiable when autograd is recording."""
    assert x.ndim == 3 and weight.shape[0] == x.shape[-1]
    if nat.compiling():
        return torch.ops.mambaqc.causal_conv1d_silu(x, weight, bias)
    nat.require_device("causal_conv1d_silu", x, weight)
    return _ConvSiLU.apply(x, weight, bias)


def causal_conv1d_silu_step_(x: torch.Tensor, tail: torch.Tensor, weight: torch.Tensor,
                             bias: torch.Tensor | None) -> torch.Tensor:
    """One recurrent step of causal_conv1d_silu: x [batch, 1, channels] (may be
    the strided first half of in_proj's output), tail [batch, k - 1, channels]
    contiguous in x's dtype, the k - 1 inputs before x (oldest first). Returns
    silu(conv) for the new row, [batch, 1, channels], equal to
    causal_conv1d_silu(cat(tail, x))[:, -1:], and updates tail in place to the
    last k - 1 inputs including x. No autograd (the decode step)."""
    B, T, C = x.shape
    K = weight.shape[-1]
    if T != 1 or weight.shape[0] != C:
        raise ValueError(f"causal_conv1d_silu_step_: x must be [batch, 1, {weight.shape[0]}], "
                         f"got {tuple(x.shape)}")
    if tail.shape != (B, K - 1, C) or tail.dtype != x.dtype or not tail.is_contiguous():
        raise ValueError(f"causal_conv1d_silu_step_: tail must be a contiguous {x.dtype} "
                         f"[{B}, {K - 1}, {C}] tensor, got {tuple(tail.shape)} {tail.dtype}")
    nat.require_device("causal_conv1d_silu_step_", x, tail, weight)
    xv, xs = _rows_view(x.detach())
    w = nat.param_f32(weight).reshape(C, K)
    b = None if bias is None else nat.param_f32(bias)
    out = torch.empty(B, 1, C, device=x.device, dtype=x.dtype)
    nat.call("mqc_causal_conv_silu_step", xv, xv.data_ptr(), xs, tail.data_ptr(), w.data_ptr(),
             nat.ptr(b), out.data_ptr(), B, C, K, nat.dtype_code(xv), nat.stream_of(xv))
    return out
