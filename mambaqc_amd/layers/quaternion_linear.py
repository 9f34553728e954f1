"""Linear maps between real and quaternion feature spaces.

Same parameters, initialisation and forward semantics as
mambaqc/layers/quaternion_linear.py:16-266, so state dicts and seeded weights
are interchangeable with the reference. The maps are dense GEMMs and run as
torch F.linear (hipBLASLt on MI355X); the quaternion layout is a view:
    real -> quaternion: [..., in] @ W^T -> [..., out/4, 4]   (+ bias [out/4, 4])
    quaternion -> real: [..., n, 4] -> [..., 4n] @ W^T       (+ bias [out])
    quaternion -> quaternion: the real block map of the flattened components.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

_KINDS = ("real", "quaternion")


class QuaternionLinear(nn.Module):
    def __init__(self, in_features: int, out_features: int, input_type: str = "real",
                 output_type: str = "quaternion", bias: bool = True):
        super().__init__()
        assert input_type in _KINDS
        assert output_type in _KINDS
        if input_type == "quaternion":
            assert in_features % 4 == 0, f"in_features must be divisible by 4, got {in_features}"
        if output_type == "quaternion":
            assert out_features % 4 == 0, f"out_features must be divisible by 4, got {out_features}"
        self.in_features = in_features
        self.out_features = out_features
        self.input_type = input_type
        self.output_type = output_type

        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        # Fan terms count quaternion features once (reference :96-119).
        fan_in = in_features // 4 if input_type == "quaternion" else in_features
        fan_out = out_features // 4 if output_type == "quaternion" else out_features
        if input_type == "real" and output_type == "real":
            nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        else:
            nn.init.normal_(self.weight, mean=0.0, std=math.sqrt(2.0 / (fan_in + fan_out)))

        if bias:
            shape = (out_features // 4, 4) if output_type == "quaternion" else (out_features,)
            self.bias = nn.Parameter(torch.zeros(shape))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.input_type == "quaternion":
            x = x.reshape(*x.shape[:-2], x.shape[-2] * 4)
        if self.output_type == "real":
            return F.linear(x, self.weight, self.bias)
        out = F.linear(x, self.weight)
        out = out.view(*out.shape[:-1], self.out_features // 4, 4)
        if self.bias is not None:
            out = out + self.bias
        return out

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"input_type={self.input_type}, output_type={self.output_type}, "
                f"bias={self.bias is not None}")


class QuaternionLinearTensorCore(nn.Module):
    """Placeholder kept for API parity (reference :211-222 raises the same way)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        raise NotImplementedError("TensorCore-optimized version not yet implemented")


def real_to_quaternion_projection(in_features: int, out_quat_dim: int,
                                  bias: bool = True) -> QuaternionLinear:
    """R^in -> H^out_quat_dim. Reference: quaternion_linear.py:227-245."""
    return QuaternionLinear(in_features, out_quat_dim * 4, "real", "quaternion", bias)


def quaternion_to_real_projection(in_quat_dim: int, out_features: int,
                                  bias: bool = True) -> QuaternionLinear:
    """H^in_quat_dim -> R^out. Reference: quaternion_linear.py:248-266."""
    return QuaternionLinear(in_quat_dim * 4, out_features, "quaternion", "real", bias)
