"""GPU operator API of the quaternion SSM hot path.

Same exports as mambaqc/kernels/__init__.py:10-33, each backed by a HIP kernel
of libmambaqc_hip.so, plus the block's fused forms `ssm_forward_fused_dl`
(delta and s given) and `ssm_forward_front_dl` (from dt_proj / gate_proj outputs),
`ssm_front` (delta = softplus(dt_raw), s = sigmoid(g_raw) * x), and
`ssm_forward_fused_bc` (the B/C projections and the SSM in one launch).

The submodule `quaternion_norm` (the layer norm) is imported before the
element-wise ops so that the package attribute `quaternion_norm` ends up bound
to the |q| function, not to the submodule of the same name.
"""
from .quaternion_norm import quaternion_layer_norm_fused, QuaternionLayerNorm
from .cayley_transform import cayley_discretization_fused
from .parallel_scan import parallel_scan_quaternion
from .ssm_fused import (ssm_step_fused, ssm_forward_fused, ssm_forward_fused_dl,
                        ssm_forward_front_dl, ssm_front, ssm_forward_fused_bc)
from .quaternion_ops import (
    quaternion_multiply,
    quaternion_multiply_batched,
    quaternion_conjugate,
    quaternion_inverse,
    quaternion_norm,
)

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
    "ssm_forward_front_dl",
    "ssm_front",
    "ssm_forward_fused_bc",
]
