"""CPU oracle for the quaternion SSM hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in plain torch on CPU tensors, of the reference's sequential
(non-Triton) path of polux06/mambaqc. Each function cites the reference
file:line it follows. It is imported only by tests/, by
__graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline leg;
the mambaqc_amd package never imports it and has no CPU path of its own.

Deviations from the unmodified reference (the reference raises on these paths):
  D1  the block gates with sigmoid(z[..., :d_model]) (the reference's Lite block,
      models/quaternion_mamba2_lite_block.py:163); the full block's
      sigmoid(z) * y_real does not broadcast when expand_factor != 1
      (models/quaternion_mamba2_block.py:160-161).
  D2  B (x) S broadcasts S over d_state (what the reference GPU kernel does,
      kernels/ssm_fused.py:134-142); the CPU path's quaternion_multiply asserts
      equal shapes first (kernels/ssm_fused.py:418, kernels/quaternion_ops.py:270).

How each function is pinned (checked independently of its own formula) is
listed in tests/test_oracle.py.
"""
from .quat import (
    IDENTITY,
    hamilton,
    conjugate,
    inverse,
    norm,
    cayley_reference,
    cumprod_reference,
    ssm_step_reference,
    ssm_forward_reference,
    ssm_forward_dl_reference,
    qln_reference,
    lambda_from_params,
)
from .block import block_forward_reference
from .lm import lm_forward_reference
from .complex_pair import ssm_forward_complex

__all__ = [
    "lm_forward_reference",
    "IDENTITY",
    "hamilton",
    "conjugate",
    "inverse",
    "norm",
    "cayley_reference",
    "cumprod_reference",
    "ssm_step_reference",
    "ssm_forward_reference",
    "ssm_forward_dl_reference",
    "qln_reference",
    "lambda_from_params",
    "block_forward_reference",
    "ssm_forward_complex",
]
