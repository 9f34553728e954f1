"""GPU parity of every form of the block's SSM walk with eps above 1 on ragged
lengths: Cayley(0) = 1 / max(1, eps) is then not the identity, so a walk that
padded a ragged tile, chunk or group with zero-delta steps would decay the
state it carries. Against torch autograd through the CPU oracle in float64 with
the same eps: the whole inference walk, the time-chunked walk, and the training
walk and backward, whole and chunked. (The fused B/C walk's eps test is in
test_gpu_fused_bc.py.)"""
import pytest
import torch

import oracle
from conftest import assert_close, tol

from mambaqc_amd import kernels as K
from mambaqc_amd.kernels.ssm_fused import ssm_fused_dl_backward, ssm_fused_dl_train_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1.6


def _inputs(b, T, d, k, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    delta = torch.nn.functional.softplus(r(b, T, d) - 1).to(dtype)
    s = r(b, T, d).to(dtype)
    Bm = (r(b, T, d, k, 4) * 0.2).to(dtype)
    C = (r(b, T, d, k, 4) * 0.2).to(dtype)
    la = r(d, k) * 0.5 + 1
    li = r(d, k, 3) * 0.3
    D = torch.ones(d) + 0.1 * r(d)
    h0 = r(b, d, k, 4) * 0.5
    gy = r(b, T, d, 4).to(dtype)
    gh = r(b, d, k, 4)
    return [delta, s, Bm, C, la, li, D, h0], gy, gh


# (batch, T, d_inner, d_state): T off the 8-step prefetch groups and the checkpoint
# interval; 64 states take the four-states-per-lane walk.
CASES = [(2, 45, 6, 16), (1, 37, 4, 64), (2, 21, 130, 8)]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_walks_with_eps_above_one(case, dtype):
    b, T, d, k = case
    print(f"eps {EPS} walks {case} {dtype}", flush=True)
    ins, gy, gh = _inputs(b, T, d, k, seed=sum(case), dtype=dtype)
    ref_in = [t.double().requires_grad_() for t in ins]
    yr, hr = oracle.ssm_forward_dl_reference(*ref_in[:7], eps=EPS, h0=ref_in[7],
                                             return_state=True)
    ((yr * gy.double()).sum() + (hr * gh.double()).sum()).backward()
    dev_in = [t.to(DEV) for t in ins]
    with torch.no_grad():
        for L in (None, 16):
            y, h = K.ssm_forward_fused_dl(*dev_in[:7], eps=EPS, h0=dev_in[7], return_state=True,
                                          chunk_len=L if L is not None else 1 << 30)
            assert_close(y, yr, tol(dtype), f"y chunk_len={L}")
            assert_close(h, hr, tol(dtype), f"h_last chunk_len={L}")
    names = ["d_delta", "d_s", "dB", "dC", "dLambda_alpha", "dLambda_imag", "dD", "dh0"]
    ckpt = 4 if dtype == torch.float32 else 8
    for L in (1 << 30, 2 * ckpt):
        y, hl, saved = ssm_fused_dl_train_forward(*dev_in[:7], h0=dev_in[7], eps=EPS,
                                                  chunk_len=L)
        assert_close(y, yr, tol(dtype), f"train y L{L}")
        assert_close(hl, hr, tol(dtype), f"train h_last L{L}")
        grads = ssm_fused_dl_backward(saved, gy.to(DEV), gh.to(DEV), eps=EPS, chunk_len=L)
        for name, got, r in zip(names, grads, ref_in):
            assert_close(got, r.grad, tol(dtype), f"{name} L{L}")
