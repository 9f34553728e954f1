"""GPU tests of DecodeGraph: the recurrent decode step of the LM captured as a
HIP graph. Every replay is checked against the same step run eagerly, with
eager work and synchronisations between the replays (a graph whose nodes
misbehave on later replays shows up on the second or third)."""
import pytest
import torch

import mambaqc_amd
from mambaqc_amd.lm import DecodeGraph

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # (vocab, d_model, n_layers, d_state, expand, dtype, batch)
    (37, 16, 2, 4, 2, torch.float32, 2),
    (301, 64, 3, 16, 2, torch.bfloat16, 3),
]


def _lm(vocab, dm, nl, ds, ex, dtype, seed=0):
    torch.manual_seed(seed)
    lm = mambaqc_amd.QuaternionMamba2(vocab, d_model=dm, n_layers=nl, d_state=ds, d_conv=4,
                                      expand_factor=ex)
    return lm.to(DEV).to(dtype).eval()


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"dm{c[1]}_l{c[2]}_s{c[3]}_{str(c[5])[6:]}")
def test_decode_graph_replays_equal_eager(case):
    vocab, dm, nl, ds, ex, dtype, batch = case
    lm = _lm(vocab, dm, nl, ds, ex, dtype)
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, vocab, (batch, 9), generator=g).to(DEV)
    with torch.no_grad():
        _, states = lm.forward_with_state(prompt)
        before = [(t.clone(), h.clone()) for t, h in states]
        graph = DecodeGraph(lm, states)
        # Building the graph leaves the caller's states as they were.
        for (t, h), (t0, h0) in zip(states, before):
            assert torch.equal(t, t0) and torch.equal(h, h0)
        eager_states = states
        for step in range(6):
            tok = torch.randint(0, vocab, (batch, 1), generator=g).to(DEV)
            want, eager_states = lm._forward_with_state(tok, eager_states)
            got = graph.step(tok)
            torch.cuda.synchronize()
            assert got.shape == (batch, 1, vocab)
            assert torch.equal(got, want), f"replay {step}: max diff {(got - want).abs().max()}"
            for i, ((tg, hg), (te, he)) in enumerate(zip(graph.states, eager_states)):
                assert torch.equal(tg, te), f"replay {step} layer {i} conv tail"
                assert torch.equal(hg, he), f"replay {step} layer {i} SSM state"
            # Unrelated eager work between replays.
            lm(prompt)
            torch.cuda.synchronize()


def test_generate_with_graph_same_tokens():
    """generate(use_graph=True) gives the tokens of the eager decode loop, greedy
    (top_k=1) and sampled from the same seed."""
    lm = _lm(301, 64, 3, 16, 2, torch.bfloat16, seed=5)
    prompt = torch.randint(0, 301, (2, 11), generator=torch.Generator().manual_seed(6)).to(DEV)
    eager = lm.generate(prompt, max_new_tokens=10, top_k=1)
    graphed = lm.generate(prompt, max_new_tokens=10, top_k=1, use_graph=True)
    assert torch.equal(eager, graphed)
    torch.manual_seed(7)
    eager = lm.generate(prompt, max_new_tokens=8, temperature=0.9, top_k=50, top_p=0.95)
    torch.manual_seed(7)
    graphed = lm.generate(prompt, max_new_tokens=8, temperature=0.9, top_k=50, top_p=0.95,
                          use_graph=True)
    assert torch.equal(eager, graphed)
