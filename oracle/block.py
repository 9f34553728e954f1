"""QuaternionMamba2Block forward restated on CPU — TEST INFRASTRUCTURE ONLY.

models/quaternion_mamba2_block.py:124-230 with deviations D1 and D2
(oracle/__init__.py). Takes the block's state_dict, so any implementation
with the reference's parameter names can be checked against it.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .quat import qln_reference, ssm_forward_dl_reference


def block_forward_reference(sd: dict, x: torch.Tensor, d_state: int, d_conv: int = 4,
                            eps_cayley: float = 1e-6, eps_norm: float = 1e-5) -> torch.Tensor:
    """x: [b, T, d_model] (CPU) -> [b, T, d_model].

    Differentiable in x and in every state-dict entry that requires grad (the
    backward's oracle is torch autograd through this function).
    """
    sd = {k: v.cpu().to(x.dtype) for k, v in sd.items()}
    b, T, d_model = x.shape
    # in_proj + chunk (:137-138)
    xz = F.linear(x, sd["in_proj.weight"], sd.get("in_proj.bias"))
    x_in, z = xz.chunk(2, dim=-1)
    D = x_in.shape[-1]
    # causal depthwise conv (layers/causal_conv1d.py:68-91) + SiLU (:141-144)
    xc = F.pad(x_in.transpose(1, 2), (d_conv - 1, 0))
    xc = F.conv1d(xc, sd["conv1d.conv.weight"], sd.get("conv1d.conv.bias"), groups=D)
    x_act = F.silu(xc.transpose(1, 2))
    # _ssm_forward (:168-230)
    delta = F.softplus(F.linear(x_act, sd["dt_proj.weight"], sd["dt_proj.bias"]))
    Bq = F.linear(x_act, sd["B_proj.weight"]).view(b, T, D, d_state, 4)
    Cq = F.linear(x_act, sd["C_proj.weight"]).view(b, T, D, d_state, 4)
    s = torch.sigmoid(F.linear(x_act, sd["gate_proj.weight"])) * x_act
    y = ssm_forward_dl_reference(delta, s, Bq, Cq, sd["Lambda_alpha"], sd["Lambda_imag"],
                                 sd["D"], eps=eps_cayley)
    # QLN (:154), out_proj (:157, layers/quaternion_linear.py:163-172)
    y = qln_reference(y, sd["norm.gamma"], sd["norm.beta"], eps=eps_norm)
    y_real = F.linear(y.reshape(b, T, D * 4), sd["out_proj.weight"], sd.get("out_proj.bias"))
    # gate (D1) + residual (:160-164)
    return x + torch.sigmoid(z[..., :d_model]) * y_real
