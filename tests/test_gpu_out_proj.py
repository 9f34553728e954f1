"""GPU parity of the fused output step (mqc_out_proj_gate_fwd, block.out_proj_gate):
x + sigmoid(z[..., :d_model]) * bf16(y W^T + bias), against float64 from the same
bf16 operands (the projection rounded to bf16 as the kernel and torch's GEMM store
it) and against the unfused path (torch's F.linear, then mqc_out_gate_fwd)."""
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_close

import mambaqc_amd
from mambaqc_amd import _native as nat
from mambaqc_amd.block import out_gate, out_proj_gate, out_proj_gate_eligible

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _operands(rows, d_model, d_inner, bias, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device=DEV)
    x = r(rows, d_model).to(BF)
    xz = r(rows, 2 * d_inner).to(BF)
    z = xz[:, d_inner:]  # the gate half of in_proj's output, read in place
    y = r(rows, d_inner, 4).to(BF)
    w = (r(d_model, 4 * d_inner) * (4 * d_inner) ** -0.5).to(BF)
    b = (r(d_model) * 0.1).to(BF) if bias else None
    return x, z, y, w, b


def _reference(x, z, y, w, b):
    yr = y.double().reshape(y.shape[0], -1) @ w.double().t()
    if b is not None:
        yr = yr + b.double()
    yr = yr.to(BF).double()  # the projection's output dtype
    d = x.shape[-1]
    return x.double() + torch.sigmoid(z[:, :d].double()) * yr


@pytest.mark.parametrize("rows,d_model,d_inner,bias", [
    (8192, 768, 1536, False),   # the headline block's output step
    (300, 200, 208, True),      # ragged token and output tiles, K = 832
    (1024, 64, 128, False),     # config 1's width (one partial output tile)
    (129, 96, 96, True),        # one token past a tile, K = 384
])
def test_out_proj_gate_vs_float64_and_unfused(rows, d_model, d_inner, bias):
    print(f"out_proj_gate rows={rows} d_model={d_model} d_inner={d_inner} bias={bias}", flush=True)
    x, z, y, w, b = _operands(rows, d_model, d_inner, bias, seed=rows + d_model)
    assert out_proj_gate_eligible(x, z, y, w, b)
    with torch.no_grad():
        got = out_proj_gate(x, z, y, w, b)
        unfused = out_gate(x, z, F.linear(y.reshape(rows, -1), w, b))
    assert got.dtype == BF and got.shape == x.shape
    want = _reference(x, z, y, w, b)
    assert_close(got, want, 2e-2, "fused output step vs float64")
    assert_close(got, unfused, 2e-2, "fused output step vs unfused")
    # The same gate arithmetic on bf16 inputs: most outputs agree bit for bit, the rest
    # where the two GEMMs' fp32 sums round y_real differently.
    same = (got == unfused).float().mean().item()
    assert same > 0.9, same


def test_out_proj_gate_rejects_what_it_cannot_run():
    x, z, y, w, b = _operands(64, 72, 16, False, seed=1)
    assert not out_proj_gate_eligible(x.float(), z.float(), y.float(), w.float(), None)
    assert not out_proj_gate_eligible(x[:, :60], z, y, w[:60], None)  # d_model % 8
    with pytest.raises(ValueError):
        out_proj_gate(x.float(), z.float(), y.float(), w.float())
    with pytest.raises(RuntimeError):
        out_proj_gate(x, z, y, w.clone().requires_grad_())
    lib = nat.load()
    # (y, W, bias, x, z, z_row_stride, out, rows, d_model, k, dtype, stream)
    P = [y.data_ptr(), w.data_ptr(), None, x.data_ptr(), z.data_ptr()]
    assert lib.mqc_out_proj_gate_fwd(*P, 32, x.data_ptr(), 64, 72, 64, 0, None) == -3
    assert lib.mqc_out_proj_gate_fwd(*P, 32, x.data_ptr(), 64, 72, 96, 1, None) == -2
    assert lib.mqc_out_proj_gate_fwd(*P, 30, x.data_ptr(), 64, 72, 64, 1, None) == -2


def test_block_output_step_fused_vs_unfused():
    """The block's output step takes the fused kernel for bf16 inference when
    fuse_out is True; against the unfused step (the default, None) on the same
    block and input."""
    torch.manual_seed(2)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16).to(DEV, BF).eval()
    x = torch.randn(2, 520, 64, generator=torch.Generator(device=DEV).manual_seed(3),
                    device=DEV).to(BF)
    with torch.no_grad():
        ref = blk(x)
        blk.fuse_out = True
        got = blk(x)
        blk.fuse_out = True
        small = blk(x[:, :7])
        blk.fuse_out = False
        small_ref = blk(x[:, :7])
    assert_close(got, ref, 2e-2, "block output step fused vs unfused")
    assert_close(small, small_ref, 2e-2, "block output step fused vs unfused, 14 rows")
