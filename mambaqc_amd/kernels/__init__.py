"""GPU operator API of the quaternion SSM hot path.

Same exports as mambaqc/kernels/__init__.py:10-33, each backed by a HIP kernel
of libmambaqc_hip.so, plus the block's fused form `ssm_forward_fused_dl`.
"""
from .quaternion_ops import (
    quaternion_multiply,
    quaternion_multiply_batched,
    quaternion_conjugate,
    quaternion_inverse,
    quaternion_norm,
)
from .cayley_transform import cayley_discretization_fused
from .parallel_scan import parallel_scan_quaternion
from .quaternion_norm import quaternion_layer_norm_fused, QuaternionLayerNorm
from .ssm_fused import ssm_step_fused, ssm_forward_fused, ssm_forward_fused_dl

__all__ = [
    "quaternion_multiply",
    "quaternion_multiply_batched",
    "quaternion_conjugate",
    "quaternion_inverse",
    "quaternion_norm",
    "cayley_discretization_fused",
    "parallel_scan_quaternion",
    "quaternion_layer_norm_fused",
    "QuaternionLayerNorm",
    "ssm_step_fused",
    "ssm_forward_fused",
    "ssm_forward_fused_dl",
]
