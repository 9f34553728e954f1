"""GPU tests of the QuaternionMamba2 LM (config 5): forward against the
reference's golden output and the CPU oracle, recurrent state and generation,
gradients, and the base preset at full size."""
import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN, assert_close

import mambaqc_amd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tiny(seed=0, d_state=4, expand=2):
    torch.manual_seed(seed)
    return mambaqc_amd.QuaternionMamba2(37, d_model=16, n_layers=2, d_state=d_state,
                                        d_conv=4, expand_factor=expand)


def test_lm_golden_s1e1():
    d = np.load(GOLDEN / "lm_s1e1.npz")
    lm = mambaqc_amd.QuaternionMamba2(37, d_model=16, n_layers=2, d_state=1, d_conv=4,
                                      expand_factor=1)
    lm.load_state_dict({k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p:")})
    lm = lm.to(DEV)
    with torch.no_grad():
        out = lm(torch.from_numpy(d["input_ids"]).to(DEV), labels=torch.from_numpy(d["labels"]).to(DEV))
    assert_close(out["logits"], torch.from_numpy(d["logits"]), 1e-4, "LM logits")
    assert_close(out["loss"], torch.from_numpy(d["loss"]), 1e-4, "LM loss")


def test_lm_vs_oracle_expand2():
    lm = _tiny()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 37, (2, 21), generator=g)
    labels = torch.randint(0, 37, (2, 21), generator=g)
    want, want_loss = oracle.lm_forward_reference(lm.state_dict(), ids, n_layers=2, d_state=4,
                                                  vocab_size=37, labels=labels)
    lm = lm.to(DEV)
    with torch.no_grad():
        out = lm(ids.to(DEV), labels=labels.to(DEV))
    assert out["logits"].shape == (2, 21, 37)
    assert_close(out["logits"], want, 1e-4, "LM logits")
    assert_close(out["loss"], want_loss, 1e-4, "LM loss")


def test_lm_rejects_bad_ids():
    lm = _tiny().to(DEV)
    with pytest.raises(AssertionError):
        lm(torch.tensor([[0, 37]], device=DEV))
    with pytest.raises(AssertionError):
        lm(torch.tensor([[-1, 3]], device=DEV))


def test_lm_state_pieces_equal_whole():
    """Feeding the sequence in pieces through forward_with_state gives the
    whole-sequence logits (the conv tails and SSM states carry over)."""
    lm = _tiny(seed=2).to(DEV)
    ids = torch.randint(0, 37, (3, 30), generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.no_grad():
        whole = lm(ids)["logits"]
        states, parts = None, []
        for a, b in ((0, 1), (1, 3), (3, 17), (17, 18), (18, 30)):
            logits, states = lm.forward_with_state(ids[:, a:b], states)
            parts.append(logits)
    assert_close(torch.cat(parts, 1), whole, 1e-4, "pieces vs whole")


def test_lm_state_pieces_equal_whole_bf16():
    """As above in bf16 over a longer walk (T 260, one single-token piece): the
    recurrent state crosses each call in fp32, so the pieces differ from the
    whole only by the GEMMs' rounding of each token, not by a state rounded
    to 16 bits at every boundary."""
    lm = _tiny(seed=8, d_state=16).to(DEV).to(torch.bfloat16)
    ids = torch.randint(0, 37, (2, 260), generator=torch.Generator().manual_seed(9)).to(DEV)
    with torch.no_grad():
        whole = lm(ids)["logits"]
        states, parts = None, []
        for a, b in ((0, 100), (100, 101), (101, 260)):
            logits, states = lm.forward_with_state(ids[:, a:b], states)
            parts.append(logits)
    assert all(st[1].dtype == torch.float32 for st in states)
    assert_close(torch.cat(parts, 1), whole, 2e-2, "bf16 pieces vs whole")


def test_generate_matches_full_recompute():
    """Recurrent generation gives the tokens of the reference's rule (full
    forward over the whole sequence per new token); greedy via top_k=1."""
    lm = _tiny(seed=4).to(DEV)
    prompt = torch.randint(0, 37, (2, 7), generator=torch.Generator().manual_seed(5)).to(DEV)
    out = lm.generate(prompt, max_new_tokens=12, top_k=1)
    ids = prompt
    with torch.no_grad():
        for _ in range(12):
            nxt = lm(ids)["logits"][:, -1].argmax(-1, keepdim=True)
            ids = torch.cat([ids, nxt], 1)
    assert torch.equal(out, ids)
    torch.manual_seed(0)
    sampled = lm.generate(prompt, max_new_tokens=5, temperature=0.8, top_k=10, top_p=0.9)
    assert sampled.shape == (2, 12) and torch.equal(sampled[:, :7], prompt)
    assert int(sampled.min()) >= 0 and int(sampled.max()) < 37


def test_lm_backward_vs_oracle():
    lm = _tiny(seed=6)
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 37, (2, 13), generator=g)
    labels = torch.randint(0, 37, (2, 13), generator=g)
    sd = {k: v.detach().double().requires_grad_(True) for k, v in lm.state_dict().items()}
    _, loss_ref = oracle.lm_forward_reference(sd, ids, n_layers=2, d_state=4, vocab_size=37,
                                              labels=labels, dtype=torch.float64)
    loss_ref.backward()
    lm = lm.to(DEV)
    lm(ids.to(DEV), labels=labels.to(DEV))["loss"].backward()
    for name, p in lm.named_parameters():
        assert p.grad is not None, name
        assert_close(p.grad, sd[name].grad, 1e-4, f"LM d{name}")


def test_lm_base_width_vs_oracle():
    """Two layers of the base preset's width (d_model 768, d_state 64, expand 2,
    vocab 10000) in bf16 at B1 T64 against the CPU oracle in fp32 on the same
    bf16-rounded weights: the blocks at config 5's shape (the 4-state SSM
    lanes, the B/C projections' column blocks) compared with a reference, not
    with themselves."""
    torch.manual_seed(0)
    with torch.device(DEV):
        lm = mambaqc_amd.QuaternionMamba2(10000, d_model=768, n_layers=2, d_state=64,
                                          d_conv=4, expand_factor=2)
    lm = lm.to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 10000, (1, 64), generator=g)
    print("LM base width, 2 layers, B1 T64, bf16", flush=True)
    with torch.inference_mode():
        got = lm(ids.to(DEV))["logits"]
    sd = {k: v.detach().float().cpu() for k, v in lm.state_dict().items()}
    del lm
    want, _ = oracle.lm_forward_reference(sd, ids, n_layers=2, d_state=64, vocab_size=10000)
    assert got.shape == want.shape == (1, 64, 10000)
    assert_close(got, want, 2e-2, "LM logits, base width (bf16 vs fp32 oracle)")


def test_lm_base_config5_forward():
    """Config 5: the base preset (12 layers, d_model 768, d_state 64; 14.66 B
    parameters) in bf16, B4 T2048, vocab 10000. Logits are finite, and causal:
    changing the last token leaves every earlier position's logits unchanged; and the
    blocks' fused B/C path (their default here) agrees with the unfused one through
    all 12 layers."""
    torch.manual_seed(0)
    with torch.device(DEV):
        lm = mambaqc_amd.quaternion_mamba2_base(10000)
    lm = lm.to(torch.bfloat16).eval()
    g = torch.Generator(device=DEV).manual_seed(0)
    ids = torch.randint(0, 10000, (4, 2048), generator=g, device=DEV)
    with torch.inference_mode():
        logits = lm(ids)["logits"]
        assert logits.shape == (4, 2048, 10000) and logits.dtype == torch.bfloat16
        assert torch.isfinite(logits).all()
        ids2 = ids.clone()
        ids2[:, -1] = (ids2[:, -1] + 1) % 10000
        logits2 = lm(ids2)["logits"]
    assert_close(logits2[:, :-1], logits[:, :-1], 1e-3, "causality")
    assert (logits2[:, -1] - logits[:, -1]).abs().max() > 0
    del logits2
    blocks = [m for m in lm.modules() if isinstance(m, mambaqc_amd.QuaternionMamba2Block)]
    assert len(blocks) == 12
    for blk in blocks:
        blk.fuse_bc = False
    with torch.inference_mode():
        unfused = lm(ids)["logits"]
    for blk in blocks:
        blk.fuse_bc = None
    assert_close(logits, unfused, 2e-2, "config 5 logits, fused B/C vs unfused")
