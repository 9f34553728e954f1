"""GPU parity of the time-chunked training walk and backward
(mqc_ssm_fused_fwd_train_chunked, mqc_ssm_fused_bwd_chunked): against torch
autograd through the CPU oracle in float64, against the whole walk and
backward on the same operands, and through the autograd path where the
library chunks by itself (small batch, few states)."""
import pytest
import torch

import oracle
from conftest import assert_close, tol

from mambaqc_amd import kernels as K
from mambaqc_amd.kernels.ssm_fused import (ssm_fused_dl_backward, ssm_fused_dl_train_forward,
                                           train_chunk_len)

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
# (batch, T, d_inner, d_state): ragged last chunks, d_state below a wave segment.
CASES = [(1, 300, 12, 16), (2, 257, 20, 8), (1, 200, 3, 64), (1, 1001, 6, 4)]


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


def _chunk_lens(dtype):
    return (20, 64) if dtype == torch.float32 else (24, 64)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("dtype", DTYPES)
def test_chunked_train_vs_oracle(case, dtype):
    b, T, d, k = case
    ins, gy, gh = _inputs(b, T, d, k, seed=sum(case), dtype=dtype)
    ref_in = [t.double().requires_grad_() for t in ins]
    yr, hr = oracle.ssm_forward_dl_reference(*ref_in[:7], h0=ref_in[7], return_state=True)
    ((yr * gy.double()).sum() + (hr * gh.double()).sum()).backward()
    dev_in = [t.to(DEV) for t in ins]
    for L in _chunk_lens(dtype):
        y, hl, saved = ssm_fused_dl_train_forward(*dev_in[:7], h0=dev_in[7], chunk_len=L)
        assert_close(y, yr, tol(dtype), f"y {case} {dtype} L{L}")
        assert_close(hl, hr, tol(dtype), f"h_last {case} {dtype} L{L}")
        grads = ssm_fused_dl_backward(saved, gy.to(DEV), gh.to(DEV), chunk_len=L)
        names = ["d_delta", "d_s", "dB", "dC", "dLambda_alpha", "dLambda_imag", "dD", "dh0"]
        for name, got, r in zip(names, grads, ref_in):
            assert_close(got, r.grad, tol(dtype), f"{name} {case} {dtype} L{L}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_chunked_train_vs_whole(dtype):
    """Same operands, whole against chunked: the checkpoints (and so the
    states) agree to fp32 rounding, and so do all gradients; without h0 and
    dh_last as well."""
    b, T, d, k = 1, 520, 40, 16
    ins, gy, gh = _inputs(b, T, d, k, seed=5, dtype=dtype)
    dev_in = [t.to(DEV) for t in ins]
    for use_state in (True, False):
        h0 = dev_in[7] if use_state else None
        ghd = gh.to(DEV) if use_state else None
        yw, hw, sw = ssm_fused_dl_train_forward(*dev_in[:7], h0=h0, chunk_len=1 << 30)
        yc, hc, sc = ssm_fused_dl_train_forward(*dev_in[:7], h0=h0, chunk_len=64)
        assert_close(yc, yw, tol(dtype), "y")
        assert_close(hc, hw, 1e-5, "h_last")
        assert_close(sc[-1], sw[-1], 1e-5, "checkpoints")
        gw = ssm_fused_dl_backward(sw, gy.to(DEV), ghd, chunk_len=1 << 30)
        gc = ssm_fused_dl_backward(sw, gy.to(DEV), ghd, chunk_len=64)
        names = ["d_delta", "d_s", "dB", "dC", "dLambda_alpha", "dLambda_imag", "dD", "dh0"]
        for name, a, w in zip(names, gc, gw):
            if w is None:
                assert a is None, name
                continue
            assert_close(a, w, 1e-4 if a.dtype == torch.float32 else tol(dtype),
                         f"{name} {dtype} state={use_state}")


def test_autograd_chunks_by_itself():
    """Through ssm_forward_fused_dl's autograd path at batch 1 with few states
    the library picks chunks; gradients against the oracle."""
    b, T, d, k = 1, 256, 4, 16
    dtype = torch.bfloat16
    assert train_chunk_len(b, T, d, k, dtype) < T
    ins, gy, gh = _inputs(b, T, d, k, seed=17, dtype=dtype)
    got_in = [t.to(DEV).requires_grad_() for t in ins]
    y, hl = K.ssm_forward_fused_dl(*got_in[:7], h0=got_in[7], return_state=True)
    ((y.float() * gy.to(DEV).float()).sum() + (hl * gh.to(DEV)).sum()).backward()
    ref_in = [t.double().requires_grad_() for t in ins]
    yr, hr = oracle.ssm_forward_dl_reference(*ref_in[:7], h0=ref_in[7], return_state=True)
    ((yr * gy.double()).sum() + (hr * gh.double()).sum()).backward()
    for name, a, r in zip(["d_delta", "d_s", "dB", "dC", "dLa", "dLi", "dD", "dh0"], got_in,
                          ref_in):
        assert_close(a.grad, r.grad, tol(dtype), name)
