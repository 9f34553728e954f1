"""mambaqc_amd — the Quaternion Mamba-2 SSM hot path on AMD MI355X (gfx950).

Drop-in for the reference package's hot path (polux06/mambaqc):
  mambaqc_amd.kernels   cayley_discretization_fused, parallel_scan_quaternion,
                        quaternion_multiply (+ conjugate/inverse/norm),
                        ssm_step_fused, ssm_forward_fused, quaternion_layer_norm_fused
  mambaqc_amd.layers    QuaternionLinear, QuaternionLayerNorm, CausalConv1d
  mambaqc_amd           QuaternionMamba2Block, QuaternionMamba2 (+ presets)
  torch.ops.mambaqc.*   the same kernels as registered torch operators with fake
                        kernels and autograd formulas (mambaqc_amd.ops)
All compute of the quaternion path runs in libmambaqc_hip.so (hand-written
HIP, C ABI in include/mambaqc_hip.h); there is no CPU fallback.
"""
__version__ = "0.1.0"

from .block import QuaternionMamba2Block, out_gate
from .lm import (
    QuaternionMamba2,
    quaternion_mamba2_base,
    quaternion_mamba2_large,
    quaternion_mamba2_small,
)
from . import ops  # registers torch.ops.mambaqc.*

__all__ = [
    "QuaternionMamba2",
    "QuaternionMamba2Block",
    "out_gate",
    "quaternion_mamba2_small",
    "quaternion_mamba2_base",
    "quaternion_mamba2_large",
]
