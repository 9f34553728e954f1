"""Layers (reference mambaqc/layers/__init__.py:5-13)."""
from .quaternion_linear import (
    QuaternionLinear,
    real_to_quaternion_projection,
    quaternion_to_real_projection,
)
from .quaternion_norm import QuaternionLayerNorm
from .causal_conv1d import CausalConv1d

__all__ = [
    "QuaternionLinear",
    "QuaternionLayerNorm",
    "CausalConv1d",
    "real_to_quaternion_projection",
    "quaternion_to_real_projection",
]
