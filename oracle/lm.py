"""QuaternionMamba2 LM forward restated on CPU — TEST INFRASTRUCTURE ONLY.

models/quaternion_mamba2.py:102-167: embedding -> blocks (block_forward_reference,
with deviations D1 and D2) -> LayerNorm -> head -> vocab slice -> cross-entropy.
Takes the model's state_dict; differentiable like block_forward_reference.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .block import block_forward_reference


def lm_forward_reference(sd: dict, input_ids: torch.Tensor, n_layers: int, d_state: int,
                         vocab_size: int, d_conv: int = 4, labels: torch.Tensor | None = None,
                         dtype: torch.dtype = torch.float32):
    """input_ids [b, T] (CPU) -> (logits [b, T, vocab_size], loss or None)."""
    x = F.embedding(input_ids, sd["embedding.weight"].cpu().to(dtype))       # :127
    for i in range(n_layers):                                                 # :131-132
        pre = f"layers.{i}."
        layer_sd = {k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}
        x = block_forward_reference(layer_sd, x, d_state=d_state, d_conv=d_conv)
    x = F.layer_norm(x, (x.shape[-1],), sd["norm_f.weight"].cpu().to(dtype),
                     sd["norm_f.bias"].cpu().to(dtype))                       # :135
    logits = F.linear(x, sd["lm_head.weight"].cpu().to(dtype))[..., :vocab_size]  # :138-141
    loss = None
    if labels is not None:                                                    # :144-162
        loss = F.cross_entropy(logits.reshape(-1, vocab_size), labels.reshape(-1),
                               ignore_index=-100)
    return logits, loss
