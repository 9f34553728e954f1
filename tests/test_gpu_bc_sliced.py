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
    forward slices by itself, with the width bc_slice_width gives."""
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
    # Training slices by the same rule (through _SlicedBCTrain).
    blk.bc_slice_d = None
    assert blk._bc_slice_width(x_act.clone().requires_grad_()) == 12


def _train_grads(blk, x, gy, state=None):
    params = [p for p in blk.parameters()]
    if state is None:
        y = blk(x)
        outs, grads_of = (y,), (gy,)
        ins = [x] + params
    else:
        y, (_, h) = blk.forward_with_state(x, state)
        outs, grads_of = (y, h), (gy, torch.ones_like(h))
        ins = [x, state[1]] + params
    return outs, torch.autograd.grad(outs, ins, grads_of)


@pytest.mark.parametrize("dtype,rtol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("width", [7, 128])
def test_sliced_training_equals_whole(dtype, rtol, width):
    """Training through _SlicedBCTrain (B/C per slice, recomputed in the
    backward) against whole projections: output and every gradient."""
    blk = _block(64, 16, dtype, seed=6)
    x = torch.randn(2, 70, 64, generator=torch.Generator(device=DEV).manual_seed(7),
                    device=DEV).to(dtype)
    gy = torch.randn(2, 70, 64, generator=torch.Generator(device=DEV).manual_seed(8),
                     device=DEV).to(dtype)
    blk.bc_slice_d = 0
    (yw,), gw = _train_grads(blk, x.clone().requires_grad_(), gy)
    blk.bc_slice_d = width
    (ys,), gs = _train_grads(blk, x.clone().requires_grad_(), gy)
    assert_close(ys, yw, rtol, f"sliced training forward w{width}")
    names = ["x"] + [n for n, _ in blk.named_parameters()]
    for n, a, b in zip(names, gs, gw):
        assert_close(a, b, max(rtol, 1e-4), f"sliced training grad {n} w{width}")


def test_sliced_training_frozen_projections():
    """B_proj and C_proj frozen: the sliced backward skips their weight
    gradients (None, as the whole path leaves them) and the other gradients
    still equal the whole path's."""
    blk = _block(64, 16, torch.float32, seed=11)
    blk.B_proj.weight.requires_grad_(False)
    blk.C_proj.weight.requires_grad_(False)
    g = torch.Generator(device=DEV).manual_seed(12)
    x = torch.randn(2, 40, 64, generator=g, device=DEV)
    gy = torch.randn(2, 40, 64, generator=g, device=DEV)
    res = {}
    for width in (0, 5):
        blk.bc_slice_d = width
        blk.zero_grad(set_to_none=True)
        xr = x.clone().requires_grad_()
        (blk(xr) * gy).sum().backward()
        assert blk.B_proj.weight.grad is None and blk.C_proj.weight.grad is None
        res[width] = [xr.grad] + [p.grad for p in blk.parameters() if p.requires_grad]
    for a, b in zip(res[5], res[0]):
        assert_close(a, b, 1e-4, "frozen-projection sliced grads")


def test_sliced_training_autocast_and_state():
    """fp32 parameters under fp16 autocast (the config-4 setting) and a
    recurrent state with gradients (h0 and h_last), sliced against whole."""
    blk = _block(64, 16, torch.float32, seed=9)
    g = torch.Generator(device=DEV).manual_seed(10)
    x = torch.randn(2, 50, 64, generator=g, device=DEV)
    gy = torch.randn(2, 50, 64, generator=g, device=DEV)
    tail = torch.randn(2, 3, 128, generator=g, device=DEV)
    h0 = torch.randn(2, 128, 16, 4, generator=g, device=DEV) * 0.1
    res = {}
    for width in (0, 9):
        blk.bc_slice_d = width
        with torch.autocast("cuda", dtype=torch.float16):
            res[width] = _train_grads(blk, x.clone().requires_grad_(), gy.half(),
                                      (tail, h0.clone().requires_grad_()))
    (yw, hw), gw = res[0]
    (ys, hs), gs = res[9]
    assert_close(ys, yw, 2e-2, "autocast sliced forward")
    assert_close(hs, hw, 1e-3, "autocast sliced h_last")
    names = ["x", "h0"] + [n for n, _ in blk.named_parameters()]
    for n, a, b in zip(names, gs, gw):
        assert_close(a, b, 2e-2, f"autocast sliced grad {n}")


def test_sliced_training_memory_bound():
    """Peak memory of a training step with 32-d slices stays well under the
    whole-projection step's (B, C, dB, dC at B1 T4096 d_inner 512 S64 bf16:
    2.1 GB each pair)."""
    blk = _block(256, 64, torch.bfloat16, seed=11)
    x = torch.randn(1, 4096, 256, device=DEV).to(torch.bfloat16)
    peaks = {}
    for width in (0, 32):
        blk.bc_slice_d = width
        blk.zero_grad(set_to_none=True)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        y = blk(x.clone().requires_grad_())
        y.float().pow(2).mean().backward()
        torch.cuda.synchronize()
        peaks[width] = torch.cuda.max_memory_allocated() - base
        del y
    assert peaks[32] < peaks[0] / 2, peaks
