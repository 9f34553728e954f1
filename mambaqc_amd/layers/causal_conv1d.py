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
