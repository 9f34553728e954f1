"""Write the golden fixtures under tests/golden/ from the reference's CPU code.

Run in a container where the reference is mounted (it does not travel):
    python tests/golden/make_golden.py [/root/reference]

Only functions that the mathematical checks in tests/test_oracle.py cannot pin
are imported from the reference, and only their CPU ("reference"/fallback)
paths run:
  * block_s1e1.npz   QuaternionMamba2Block forward at d_state=1, expand_factor=1
                     (the one block configuration the reference's CPU path runs
                     without raising), seed 0: parameters, input and output.
                     Pins the block's op order, the causal conv, gating and the
                     parameter-creation (RNG) order.
  * init_c1.json     seed-0 constructor of QuaternionMamba2Block(64, d_state=16,
                     d_conv=4, expand_factor=2) (config 1): per-parameter shape,
                     sha256 of the fp32 bytes, and the first/last 4 values.
  * qln.npz          quaternion_layer_norm_reference on rows with tiny norms,
                     where the placement of the two eps terms matters.
  * cayley.npz       cayley_discretization_reference including inputs where the
                     eps clamp of the inverse engages (|1 - z/2|^2 <= eps).
  * lm_s1e1.npz      QuaternionMamba2 LM (vocab 37, d_model 16, 2 layers, d_state 1,
                     expand 1; the LM configuration the reference's CPU path runs),
                     seed 0: parameters, input ids, labels, logits and loss. Pins
                     embedding, block stacking, final LayerNorm, head, vocab slice
                     and the loss.
  * init_lm.json     seed-0 constructor of QuaternionMamba2(37, d_model=16, n_layers=2,
                     d_state=4, expand_factor=2): per-parameter shape and sha256 (the
                     LM re-initialises nn.Linear / nn.Embedding weights in module
                     traversal order after the blocks draw theirs).
Fixtures are data only (npz without pickles, JSON).

    python tests/golden/make_golden.py [/root/reference] [--only-lm]
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _param_info(module) -> dict:
    info = {}
    for k, v in module.state_dict().items():
        a = v.detach().float().contiguous().numpy()
        info[k] = {
            "shape": list(a.shape),
            "sha256": hashlib.sha256(a.tobytes()).hexdigest(),
            "head": [float(t) for t in a.reshape(-1)[:4]],
            "tail": [float(t) for t in a.reshape(-1)[-4:]],
        }
    return info


def write_lm(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from mambaqc.models.quaternion_mamba2 import QuaternionMamba2

    torch.set_num_threads(1)
    torch.manual_seed(0)
    lm = QuaternionMamba2(37, d_model=16, n_layers=2, d_state=1, d_conv=4, expand_factor=1)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 37, (2, 9), generator=g)
    labels = torch.randint(0, 37, (2, 9), generator=g)
    labels[0, 3] = -100
    with torch.no_grad():
        out = lm(ids, labels=labels)
    arrays = {"input_ids": ids.numpy(), "labels": labels.numpy(),
              "logits": out["logits"].numpy(), "loss": out["loss"].numpy()}
    for k, v in lm.state_dict().items():
        arrays["p:" + k] = v.numpy()
    np.savez(HERE / "lm_s1e1.npz", **arrays)

    torch.manual_seed(0)
    lm = QuaternionMamba2(37, d_model=16, n_layers=2, d_state=4, d_conv=4, expand_factor=2)
    (HERE / "init_lm.json").write_text(json.dumps(_param_info(lm), indent=1) + "\n")
    print("wrote lm_s1e1.npz init_lm.json")


def main(ref_root: str = "/root/reference") -> None:
    sys.path.insert(0, ref_root)
    from mambaqc.models.quaternion_mamba2_block import QuaternionMamba2Block
    from mambaqc.kernels.quaternion_norm import quaternion_layer_norm_reference
    from mambaqc.kernels.cayley_transform import cayley_discretization_reference

    torch.set_num_threads(1)

    # Block at d_state=1, expand_factor=1.
    torch.manual_seed(0)
    blk = QuaternionMamba2Block(16, d_state=1, d_conv=4, expand_factor=1)
    x = torch.randn(2, 8, 16)
    with torch.no_grad():
        out = blk(x)
    arrays = {"x": x.numpy(), "out": out.numpy()}
    for k, v in blk.state_dict().items():
        arrays["p:" + k] = v.numpy()
    np.savez(HERE / "block_s1e1.npz", **arrays)

    # Seeded init at config 1.
    torch.manual_seed(0)
    blk = QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    info = {}
    for k, v in blk.state_dict().items():
        a = v.detach().float().contiguous().numpy()
        info[k] = {
            "shape": list(a.shape),
            "sha256": hashlib.sha256(a.tobytes()).hexdigest(),
            "head": [float(t) for t in a.reshape(-1)[:4]],
            "tail": [float(t) for t in a.reshape(-1)[-4:]],
        }
    (HERE / "init_c1.json").write_text(json.dumps(info, indent=1) + "\n")

    # QLN with tiny norms.
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, 3, 7, 4, generator=g)
    q[0, 0] *= 1e-3
    q[1, 2, :3] *= 1e-4
    gamma = torch.rand(7, generator=g) + 0.5
    beta = torch.randn(7, 4, generator=g) * 0.1
    out = quaternion_layer_norm_reference(q, gamma, beta, eps=1e-5)
    np.savez(HERE / "qln.npz", q=q.numpy(), gamma=gamma.numpy(), beta=beta.numpy(),
             out=out.numpy(), eps=np.float32(1e-5))

    # Cayley, including the clamp: z = (2, 0, 0, 0) gives |1 - z/2|^2 = 0.
    z = torch.randn(1, 2, 3, 4, 4, generator=g)
    z[0, 0, 0, 0] = torch.tensor([2.0, 0.0, 0.0, 0.0])
    z[0, 0, 0, 1] = torch.tensor([2.0, 1e-3, 0.0, 0.0])
    z[0, 0, 1, 0] = torch.tensor([1.999, 0.0, 0.0, 0.0])
    z[0, 1, 2, 3] = torch.tensor([-3.0, 0.5, -0.25, 2.0])
    qz = cayley_discretization_reference(z, eps=1e-6)
    np.savez(HERE / "cayley.npz", z=z.numpy(), q=qz.numpy(), eps=np.float32(1e-6))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")), "init_c1.json")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    if "--only-lm" in sys.argv:
        write_lm(*args)
    else:
        main(*args)
        write_lm(*args)
