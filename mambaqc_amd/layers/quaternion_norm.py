"""Import path mambaqc.layers.quaternion_norm (reference layers/quaternion_norm.py:1-17)."""
from ..kernels.quaternion_norm import QuaternionLayerNorm, quaternion_layer_norm_fused

__all__ = ["QuaternionLayerNorm", "quaternion_layer_norm_fused"]
