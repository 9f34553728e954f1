"""GPU tests of the in-place recurrent decode step: the conv step kernel
(mqc_causal_conv_silu_step), the SSM walk that writes its final state over its
initial one, and the block / LM steps built on them, each against the
out-of-place path it replaces (same kernels and order of operations, so equal
bit for bit) and, through it, the oracle-checked forward."""
import pytest
import torch

import mambaqc_amd
from mambaqc_amd.kernels import ssm_fused as sf
from mambaqc_amd.layers.causal_conv1d import causal_conv1d_silu, causal_conv1d_silu_step_

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,C,K", [(1, 8, 4), (3, 37, 4), (2, 64, 1), (2, 20, 2), (4, 1536, 4),
                                   (1, 9, 8)])
def test_conv_step_equals_conv_of_concatenation(dtype, B, C, K):
    g = torch.Generator(device=DEV).manual_seed(B * 100 + C + K)
    xz = torch.randn(B, 1, 2 * C, generator=g, device=DEV).to(dtype)
    x = xz[..., :C]  # strided rows, as the block's in_proj half
    tail = torch.randn(B, K - 1, C, generator=g, device=DEV).to(dtype)
    w = torch.randn(C, 1, K, generator=g, device=DEV) * 0.3
    bias = torch.randn(C, generator=g, device=DEV) * 0.1
    xc = torch.cat([tail, x], dim=1)
    want = causal_conv1d_silu(xc, w, bias)[:, -1:]
    want_tail = xc[:, 1:].clone()
    t = tail.clone()
    got = causal_conv1d_silu_step_(x, t, w, bias)
    assert torch.equal(got, want)
    assert torch.equal(t, want_tail)
    got2 = causal_conv1d_silu_step_(x, tail.clone(), w, None)
    assert torch.equal(got2, causal_conv1d_silu(xc, w, None)[:, -1:])


def test_conv_step_rejects_bad_tails():
    x = torch.randn(2, 1, 16, device=DEV)
    w = torch.randn(16, 1, 4, device=DEV)
    for tail in (torch.randn(2, 2, 16, device=DEV), torch.randn(2, 3, 16, device=DEV).half(),
                 torch.randn(2, 16, 3, device=DEV).transpose(1, 2)):
        with pytest.raises(ValueError):
            causal_conv1d_silu_step_(x, tail, w, None)
    with pytest.raises(ValueError):
        causal_conv1d_silu_step_(torch.randn(2, 2, 16, device=DEV), torch.randn(2, 3, 16, device=DEV),
                                 w, None)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("b,T,d,k", [(4, 1, 48, 16), (2, 3, 20, 5), (1, 1, 1536, 64)])
def test_ssm_state_in_place_equals_out_of_place(dtype, b, T, d, k):
    g = torch.Generator(device=DEV).manual_seed(T * 7 + d)
    r = lambda *s: torch.randn(*s, generator=g, device=DEV)
    dt_raw, g_raw, x = r(b, T, d).to(dtype), r(b, T, d).to(dtype), r(b, T, d).to(dtype)
    Bm, C = (r(b, T, d, k, 4) * 0.2).to(dtype), (r(b, T, d, k, 4) * 0.2).to(dtype)
    la, li, D = r(d, k) * 0.5 + 1, r(d, k, 3) * 0.3, 1 + 0.1 * r(d)
    h0 = r(b, d, k, 4) * 0.5
    with torch.no_grad():
        yw, hw = sf.ssm_forward_front_dl(dt_raw, g_raw, x, Bm, C, la, li, D, h0=h0,
                                         return_state=True)
        h = h0.clone()
        y = sf.ssm_forward_front_dl_state_(dt_raw, g_raw, x, Bm, C, la, li, D, h)
    assert torch.equal(y, yw)
    assert torch.equal(h, hw)


def test_ssm_state_in_place_refuses_autograd_and_bad_state():
    d, k = 8, 4
    args = [torch.randn(1, 1, d, device=DEV) for _ in range(3)]
    args += [torch.randn(1, 1, d, k, 4, device=DEV) for _ in range(2)]
    args += [torch.randn(d, k, device=DEV), torch.randn(d, k, 3, device=DEV), torch.ones(d, device=DEV)]
    h = torch.zeros(1, d, k, 4, device=DEV)
    with pytest.raises(RuntimeError):
        sf.ssm_forward_front_dl_state_(*args[:2], args[2].requires_grad_(), *args[3:], h)
    args[2] = args[2].detach()
    with pytest.raises(ValueError):
        sf.ssm_forward_front_dl_state_(*args, h.half())


def _block(dtype, seed=0):
    torch.manual_seed(seed)
    with torch.device(DEV):
        blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    return blk.to(dtype).eval()


@pytest.mark.parametrize("dtype", DTYPES)
def test_block_step_state_equals_forward_with_state(dtype):
    blk = _block(dtype)
    g = torch.Generator(device=DEV).manual_seed(1)
    prompt = torch.randn(3, 11, 64, generator=g, device=DEV).to(dtype)
    toks = torch.randn(3, 6, 64, generator=g, device=DEV).to(dtype)
    with torch.no_grad():
        _, st = blk.forward_with_state(prompt)
        tail, h = st[0].contiguous(), st[1].clone()
        for i in range(toks.shape[1]):
            x = toks[:, i:i + 1]
            want, st = blk.forward_with_state(x, st)
            got = blk.step_state_(x, (tail, h))
            assert torch.equal(got, want), i
            assert torch.equal(tail, st[0]) and torch.equal(h, st[1]), i


def test_lm_step_state_equals_forward_with_state():
    torch.manual_seed(0)
    with torch.device(DEV):
        lm = mambaqc_amd.QuaternionMamba2(53, d_model=32, n_layers=3, d_state=8).to(torch.bfloat16)
    lm.eval()
    g = torch.Generator(device=DEV).manual_seed(2)
    ids = torch.randint(0, 53, (2, 9), generator=g, device=DEV)
    with torch.no_grad():
        _, states = lm.forward_with_state(ids)
        mine = [(t.contiguous(), h.clone()) for t, h in states]
        for i in range(5):
            tok = torch.randint(0, 53, (2, 1), generator=g, device=DEV)
            want, states = lm._forward_with_state(tok, states)
            got = lm._step_state_(tok, mine)
            assert torch.equal(got, want), i
