"""GPU tests of the block's d-sliced B/C path (inference): B and C computed a
slice of d's at a time into reused buffers, each slice's SSM run from them.
Checked against the whole-projection path, against the oracle (including the
headline width), through the recurrent state, and for the automatic rule."""
import pytest
import torch

import oracle
from conftest import assert_close

import mambaqc_amd
from mambaqc_amd import block as block_mod

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _block(dm, ds, dtype, seed=0):
    torch.manual_seed(seed)
    with torch.device(DEV):
        blk = mambaqc_amd.QuaternionMamba2Block(dm, d_state=ds, d_conv=4, expand_factor=2)
    return blk.to(dtype)


@pytest.mark.parametrize("dtype,rtol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("width", [1, 7, 128, 500])
def test_sliced_equals_whole(dtype, rtol, width):
    """Ragged last slice (7 into 128), one d per slice, one slice, and a width
    above d_inner, against whole projections and against the oracle."""
    blk = _block(64, 16, dtype)
    x = torch.randn(2, 300, 64, generator=torch.Generator(device=DEV).manual_seed(1),
                    device=DEV).to(dtype)
    with torch.no_grad():
        blk.bc_slice_d = 0
        whole = blk(x)
        blk.bc_slice_d = width
        got = blk(x)
    assert got.dtype == dtype and got.shape == whole.shape
    assert_close(got, whole, rtol, f"sliced w{width} vs whole")
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.float().cpu(), d_state=16)
    assert_close(got, want, max(rtol, 1e-4), f"sliced w{width} vs oracle")


def test_sliced_headline_width_bf16_vs_oracle():
    """d_model 768, d_state 64, expand 2 (d_inner 1536) in bf16 at B4 T256 with
    96 d's per slice (16 slices, each slice's SSM chunked by the library's
    rule) against the oracle in fp32 on the same bf16-rounded weights."""
    blk = _block(768, 64, torch.bfloat16, seed=11)
    x = torch.randn(4, 256, 768, generator=torch.Generator(device=DEV).manual_seed(12),
                    device=DEV).to(torch.bfloat16)
    blk.bc_slice_d = 96
    with torch.no_grad():
        got = blk(x)
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.float().cpu(), d_state=64)
    assert_close(got, want, 2e-2, "sliced block d768 s64 e2 bf16")


@pytest.mark.parametrize("dtype,rtol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_sliced_state_pieces(dtype, rtol):
    """forward_with_state with sliced B/C: pieces equal the whole sequence, and
    the final state (fp32) equals the whole-projection path's."""
    blk = _block(64, 16, dtype, seed=2)
    x = torch.randn(3, 200, 64, generator=torch.Generator(device=DEV).manual_seed(4),
                    device=DEV).to(dtype)
    with torch.no_grad():
        blk.bc_slice_d = 0
        y_ref, (tail_ref, h_ref) = blk.forward_with_state(x)
        blk.bc_slice_d = 9
        y_all, (tail_all, h_all) = blk.forward_with_state(x)
        ya, st = blk.forward_with_state(x[:, :77])
        yb, (tail_b, h_b) = blk.forward_with_state(x[:, 77:], st)
    assert h_all.dtype == torch.float32
    assert_close(y_all, y_ref, rtol, "sliced y vs whole")
    assert_close(h_all, h_ref, max(rtol, 1e-5), "sliced state vs whole")
    assert torch.equal(tail_all, tail_ref)
    assert_close(torch.cat([ya, yb], 1), y_all, rtol, "sliced pieces vs whole sequence")
    assert_close(h_b, h_all, max(rtol, 1e-5), "sliced pieces state")


def test_sliced_auto_rule(monkeypatch):
    """With the whole-projection bound lowered below this input's B and C, the
    inference forward slices by itself, with the width bc_slice_width gives."""
    blk = _block(64, 16, torch.float32, seed=3)
    x = torch.randn(2, 128, 64, device=DEV)
    with torch.no_grad():
        whole = blk(x)
        bc_bytes = 2 * 2 * 128 * 128 * 16 * 4 * 4
        monkeypatch.setattr(block_mod, "BC_WHOLE_MAX_BYTES", bc_bytes - 1)
        monkeypatch.setattr(block_mod, "BC_SLICE_BYTES", bc_bytes // 10)
        x_act = torch.zeros(2, 128, 128, device=DEV)  # the SSM's input: d_inner wide
        assert blk._bc_slice_width(x_act) == block_mod.bc_slice_width(2, 128, 128, 16, 4,
                                                                      bc_bytes // 10) == 12
        got = blk(x)
        blk.bc_slice_d = 12
        forced = blk(x)
    assert torch.equal(got, forced)
    assert_close(got, whole, 1e-5, "auto-sliced vs whole")
    # Training never slices on its own.
    blk.bc_slice_d = None
    assert blk._bc_slice_width(x_act.clone().requires_grad_()) == 0
