"""GPU parity of the fused B/C projections + SSM walk (mqc_ssm_fused_bc_fwd,
kernels.ssm_forward_fused_bc) against the CPU oracle and against the unfused
path (torch's GEMMs for B and C, then mqc_ssm_fused_fwd).

The oracle side: B = x W_B^T and C = x W_C^T in fp32 from the same 16-bit
operands, rounded to their dtype (what the projections store and the fused kernel
rounds to on chip), then oracle.ssm_forward_dl_reference in float64. bf16 and fp16
tolerance 2e-2 with the atol floor of rtol * max|ref| (conftest.assert_close).
"""
import ctypes

import pytest
import torch

import oracle
from conftest import assert_close

from mambaqc_amd import _native as nat
from mambaqc_amd import kernels as K
from mambaqc_amd.kernels.ssm_fused import fused_bc_eligible

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
F16 = torch.float16


def _inputs(b, T, d, k, seed, w_std=None, dt=BF):
    g = torch.Generator(device=DEV).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device=DEV)
    w_std = 0.3 / d ** 0.5 if w_std is None else w_std
    x = r(b, T, d).to(dt)
    wb = (r(d * k * 4, d) * w_std).to(dt)
    wc = (r(d * k * 4, d) * w_std).to(dt)
    delta = torch.nn.functional.softplus(r(b, T, d) - 1).to(dt)
    s = r(b, T, d).to(dt)
    la = r(d, k) * 0.5 + 1
    li = r(d, k, 3) * 0.3
    D = 1 + 0.1 * r(d)
    h0 = r(b, d, k, 4) * 0.2
    return x, wb, wc, delta, s, la, li, D, h0


def _bc_rounded(x, w, d_slice, k):
    """B (or C) for the d's of d_slice, as the projections store it: fp32 GEMM of
    the 16-bit operands, rounded to their dtype; [b, T, n_d, k, 4] in float64 on
    the CPU."""
    b, T, d = x.shape
    rows = w.view(d, k * 4, d)[d_slice].reshape(-1, d)
    out = (x.float().reshape(-1, d) @ rows.float().t()).to(x.dtype)
    return out.double().cpu().view(b, T, -1, k, 4)


def _oracle(x, wb, wc, delta, s, la, li, D, h0, d_slice, b_slice=slice(None), eps=1e-6):
    k = la.shape[-1]
    xs = x[b_slice]
    Bq = _bc_rounded(xs, wb, d_slice, k)
    Cq = _bc_rounded(xs, wc, d_slice, k)
    up = lambda t: t.detach().double().cpu()
    return oracle.ssm_forward_dl_reference(
        up(delta[b_slice][:, :, d_slice]), up(s[b_slice][:, :, d_slice]), Bq, Cq,
        up(la[d_slice]), up(li[d_slice]), up(D[d_slice]), eps=eps,
        h0=None if h0 is None else up(h0[b_slice][:, d_slice]), return_state=True)


@pytest.mark.parametrize("shape", [
    (1, 256, 64, 64),    # one full tile, one K step
    (2, 512, 128, 64),   # state carried across tiles
    (3, 300, 192, 32),   # ragged last tile, one half of states, d_inner 3 x 64
    (1, 77, 64, 16),     # shorter than a tile, a ragged half (16 states)
    (2, 600, 64, 48),    # two halves, the second ragged
    (1, 300, 64, 34),    # the second half two states (one 8-row DMA group of W rows)
    (1, 1, 128, 2),      # one token, two states
])
@pytest.mark.parametrize("with_h0", [False, True])
@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_vs_oracle(shape, with_h0, dt):
    b, T, d, k = shape
    print(f"fused_bc vs oracle {shape} h0={with_h0} {dt}", flush=True)
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=sum(shape), dt=dt)
    h0 = h0 if with_h0 else None
    assert fused_bc_eligible(x, wb, wc, k)
    with torch.no_grad():
        y, h = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0, return_state=True)
    want_y, want_h = _oracle(x, wb, wc, delta, s, la, li, D, h0, slice(None))
    assert y.dtype == dt and h.dtype == torch.float32
    assert_close(y, want_y, 2e-2, f"fused y {shape}")
    assert_close(h, want_h, 2e-2, f"fused h_last {shape}")


@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_equals_unfused_path_small(dt):
    """Against the unfused path on the same weights (torch's 16-bit GEMMs, then the
    library's walk): the same recurrence on B and C that differ at most by the
    rounding of differently ordered fp32 sums."""
    b, T, d, k = 2, 700, 128, 64
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=5, dt=dt)
    with torch.no_grad():
        y, h = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0, return_state=True)
        Bq = torch.nn.functional.linear(x, wb).view(b, T, d, k, 4)
        Cq = torch.nn.functional.linear(x, wc).view(b, T, d, k, 4)
        y2, h2 = K.ssm_forward_fused_dl(delta, s, Bq, Cq, la, li, D, h0=h0, return_state=True)
    assert_close(y, y2, 2e-2, "fused vs unfused y")
    assert_close(h, h2, 2e-2, "fused vs unfused h_last")


@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_config3_full_size(dt):
    """Config 3's shape (B4 T2048 d_inner 1536 S64; bf16, and the same in fp16): the
    whole output against the unfused path on the same weights, and d-slices in every
    batch row (each (b, d) is its own workgroup; slices at both ends and in the
    middle of the launch order) against the oracle."""
    b, T, d, k = 4, 2048, 1536, 64
    print(f"fused_bc config 3 full size {dt}", flush=True)
    x, wb, wc, delta, s, la, li, D, _ = _inputs(b, T, d, k, seed=0, w_std=0.02, dt=dt)
    with torch.no_grad():
        y = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D)
        Bq = torch.nn.functional.linear(x, wb).view(b, T, d, k, 4)
        Cq = torch.nn.functional.linear(x, wc).view(b, T, d, k, 4)
        y2 = K.ssm_forward_fused_dl(delta, s, Bq, Cq, la, li, D)
        del Bq, Cq
    assert_close(y, y2, 2e-2, "C3 fused vs unfused")
    for b0, ds in ((0, slice(0, 2)), (1, slice(700, 702)), (2, slice(1000, 1001)),
                   (3, slice(1534, 1536))):
        want, _ = _oracle(x, wb, wc, delta, s, la, li, D, None, ds, slice(b0, b0 + 1))
        assert_close(y[b0:b0 + 1, :, ds], want, 2e-2, f"C3 fused slice b={b0} d={ds}")
    # Every lane at full size: y is linear in s (B and C do not depend on it), and
    # doubling is exact in floating point, so 2 s gives 2 y bit for bit; except that
    # where y rounds into fp16's subnormals (fixed spacing 2^-24) rounding 2 y and
    # doubling the rounded y may differ by that spacing.
    with torch.no_grad():
        y_2s = K.ssm_forward_fused_bc(x, wb, wc, delta, (2 * s.float()).to(dt), la, li, D)
    want_2s = (2 * y.float()).to(dt)
    normal = y.float().abs() >= torch.finfo(dt).tiny
    assert torch.equal(y_2s[normal], want_2s[normal])
    assert (y_2s.float() - want_2s.float()).abs().max().item() <= 2.0 ** -24


@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_state_in_place_and_empty(dt):
    """h_last may be h0 (each (b, d) reads its own states before it writes them),
    through the C ABI; an empty sequence copies h0 to h_last."""
    b, T, d, k = 2, 300, 64, 64
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=9, dt=dt)
    with torch.no_grad():
        y_ref, h_ref = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0,
                                              return_state=True)
    lib = nat.load()
    h = h0.clone()
    y = torch.empty_like(y_ref)
    stream = torch.cuda.current_stream().cuda_stream
    st = lib.mqc_ssm_fused_bc_fwd(x.data_ptr(), wb.data_ptr(), wc.data_ptr(), delta.data_ptr(),
                                  s.data_ptr(), la.data_ptr(), li.data_ptr(), D.data_ptr(),
                                  h.data_ptr(), y.data_ptr(), h.data_ptr(), b, T, d, k, 1e-6,
                                  nat.dtype_code(x), stream)
    assert st == 0, nat.status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref) and torch.equal(h, h_ref)
    h_out = torch.full_like(h0, float("nan"))
    st = lib.mqc_ssm_fused_bc_fwd(None, None, None, None, None, la.data_ptr(), li.data_ptr(),
                                  D.data_ptr(), h0.data_ptr(), None, h_out.data_ptr(), b, 0, d,
                                  k, 1e-6, nat.dtype_code(x), stream)
    assert st == 0, nat.status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(h_out, h0)


def test_fused_bc_rejects_what_it_cannot_run():
    x, wb, wc, delta, s, la, li, D, _ = _inputs(1, 16, 64, 4, seed=3)
    assert not fused_bc_eligible(x.float(), wb.float(), wc.float(), 4)
    assert not fused_bc_eligible(x.half(), wb, wc, 4)  # mixed 16-bit dtypes
    assert fused_bc_eligible(x.half(), wb.half(), wc.half(), 4)
    assert not fused_bc_eligible(x, wb, wc, 3)
    with pytest.raises(ValueError):
        K.ssm_forward_fused_bc(x.float(), wb.float(), wc.float(), delta, s, la, li, D)
    with pytest.raises(RuntimeError):
        K.ssm_forward_fused_bc(x, wb.requires_grad_(), wc, delta, s, la, li, D)


def test_block_forward_fused_bc_path():
    """QuaternionMamba2Block inference in bf16 takes the fused path from
    FUSED_BC_MIN_SEQ tokens on: its output against the same block with fusion off
    and against the CPU oracle of the block (fp32 on the same bf16 weights), a
    sequence fed in two pieces through forward_with_state against the whole."""
    import mambaqc_amd
    from mambaqc_amd import block as blockmod

    torch.manual_seed(0)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16).to(DEV, BF).eval()
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(2, 300, 64, generator=g, device=DEV).to(BF)
    assert x.shape[1] >= blockmod.FUSED_BC_MIN_SEQ and blk._use_fused_bc(
        torch.empty(2, 300, blk.d_inner, device=DEV, dtype=BF))
    # A batch of one fuses too (split halves); short sequences do not unless forced.
    assert blk._use_fused_bc(torch.empty(1, 300, blk.d_inner, device=DEV, dtype=BF))
    short = torch.empty(2, blockmod.FUSED_BC_MIN_SEQ - 1, blk.d_inner, device=DEV, dtype=BF)
    assert not blk._use_fused_bc(short)
    blk.fuse_bc = True
    assert blk._use_fused_bc(short)
    blk.fuse_bc = None
    with torch.no_grad():
        got = blk(x)
        blk.fuse_bc = False
        ref_unfused = blk(x)
        blk.fuse_bc = None
        out1, st = blk.forward_with_state(x[:, :260])
        out2, _ = blk.forward_with_state(x[:, 260:], st)
    assert_close(got, ref_unfused, 2e-2, "block fused vs unfused")
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.float().cpu(), d_state=16)
    assert_close(got, want, 2e-2, "block fused vs oracle")
    assert_close(torch.cat([out1, out2], 1), got, 2e-2, "fused block in pieces vs whole")


@pytest.mark.parametrize("shape,with_h0", [
    ((1, 300, 128, 64), False),   # ragged last tile, two full halves
    ((1, 600, 64, 48), True),     # the second half ragged (16 states)
    ((1, 300, 64, 34), True),     # the second half two states
    ((2, 512, 128, 64), True),    # batch 2, state carried across tiles
    ((1, 256, 64, 32), False),    # one half: the split call is the one-launch form
    ((1, 1, 64, 64), True),       # one token
])
@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_split_equals_one_launch(shape, with_h0, dt):
    """Each half of the states in a workgroup of its own, partial sums added by a
    second launch (mqc_ssm_fused_bc_fwd_split): y and h_last equal the one-launch
    form bit for bit, and the oracle to 16-bit tolerance."""
    b, T, d, k = shape
    print(f"fused_bc split {shape} h0={with_h0} {dt}", flush=True)
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=11 + sum(shape), dt=dt)
    h0 = h0 if with_h0 else None
    with torch.no_grad():
        y1, h1 = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0,
                                        return_state=True, split=False)
        y2, h2 = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0,
                                        return_state=True, split=True)
    assert torch.equal(y1, y2) and torch.equal(h1, h2)
    want_y, want_h = _oracle(x, wb, wc, delta, s, la, li, D, h0, slice(None))
    assert_close(y2, want_y, 2e-2, f"split y {shape}")
    assert_close(h2, want_h, 2e-2, f"split h_last {shape}")


def test_fused_bc_split_through_c_abi():
    """The split entry point through the C ABI: h_last may be h0 (each half's
    workgroup reads and writes only its own states), a short workspace is refused
    before any launch, and the default of ssm_forward_fused_bc splits a batch of one."""
    from mambaqc_amd.kernels import ssm_fused

    b, T, d, k = 1, 300, 64, 64
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=21)
    with torch.no_grad():
        y_ref, h_ref = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0,
                                              return_state=True, split=False)
    assert ssm_fused.FUSED_BC_SPLIT_MAX_BATCH >= 1
    lib = nat.load()
    need = lib.mqc_ssm_fused_bc_split_workspace_bytes(b, T, d, k)
    assert need == 2 * b * T * d * 16
    ws = torch.empty(need, device=DEV, dtype=torch.uint8)
    h = h0.clone()
    y = torch.empty_like(y_ref)
    stream = torch.cuda.current_stream().cuda_stream
    P = [x.data_ptr(), wb.data_ptr(), wc.data_ptr(), delta.data_ptr(), s.data_ptr(),
         la.data_ptr(), li.data_ptr(), D.data_ptr(), h.data_ptr(), y.data_ptr(), h.data_ptr(),
         b, T, d, k, 1e-6, nat.BF16]
    assert lib.mqc_ssm_fused_bc_fwd_split(*P, ws.data_ptr(), need - 16, stream) == -6
    assert lib.mqc_ssm_fused_bc_fwd_split(*P, None, need, stream) == -1
    assert torch.equal(h, h0)
    st = lib.mqc_ssm_fused_bc_fwd_split(*P, ws.data_ptr(), need, stream)
    assert st == 0, nat.status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref) and torch.equal(h, h_ref)
    with torch.no_grad():
        y_def = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0)
    assert torch.equal(y_def, y_ref)


def test_block_batch_of_one_takes_split_fused_path():
    """A batch of one with two halves of states (d_state 64) runs the split fused
    kernel inside the block: against the same block unfused, its row of a batch of
    two (one workgroup per d) and the CPU oracle of the block."""
    import mambaqc_amd

    torch.manual_seed(4)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=64).to(DEV, BF).eval()
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(2, 280, 64, generator=g, device=DEV).to(BF)
    with torch.no_grad():
        one = blk(x[:1])
        both = blk(x)
        blk.fuse_bc = False
        one_unfused = blk(x[:1])
        blk.fuse_bc = None
    # (torch's GEMMs around the SSM may tile 280 and 560 rows differently.)
    assert_close(one, both[:1], 2e-2, "split fused block vs its row of a batch of two")
    assert_close(one, one_unfused, 2e-2, "split fused block vs unfused, batch of one")
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x[:1].float().cpu(), d_state=64)
    assert_close(one, want, 2e-2, "split fused block vs oracle")


@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_split_in_time_segments(monkeypatch, dt):
    """A batch of one whose split workspace would pass FUSED_BC_SPLIT_WS_MAX is
    walked in segments of whole 256-token tiles, the fp32 state carried through
    h0 / h_last: the same y and final state as one launch, bit for bit."""
    from mambaqc_amd.kernels import ssm_fused

    b, T, d, k = 1, 700, 64, 64
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=31, dt=dt)
    with torch.no_grad():
        y1, h1 = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0,
                                        return_state=True, split=False)
        # 2 x d x 16 bytes of workspace per token: segments of 256, 256 and 188 tokens.
        monkeypatch.setattr(ssm_fused, "FUSED_BC_SPLIT_WS_MAX", 2 * d * 16 * 300)
        y2, h2 = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0,
                                        return_state=True, split=True)
        y3 = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, h0=h0, split=True)
    assert torch.equal(y1, y2) and torch.equal(h1, h2) and torch.equal(y1, y3)


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("dt", [BF, F16], ids=["bf16", "f16"])
def test_fused_bc_eps_clamp(split, dt):
    """An eps large enough that the clamp max(N, eps) of the Cayley map engages on
    the steps with small delta (N = 1 - delta a + delta^2 |Lambda|^2 / 4 >= 1 here,
    eps 1.6): the fused walk, in both forms, against the oracle with the same eps."""
    b, T, d, k = 1, 300, 64, 64
    x, wb, wc, delta, s, la, li, D, h0 = _inputs(b, T, d, k, seed=41, dt=dt)
    with torch.no_grad():
        y, h = K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, D, eps=1.6, h0=h0,
                                      return_state=True, split=split)
    want_y, want_h = _oracle(x, wb, wc, delta, s, la, li, D, h0, slice(None), eps=1.6)
    assert_close(y, want_y, 2e-2, "fused y, eps clamp")
    assert_close(h, want_h, 2e-2, "fused h_last, eps clamp")


@pytest.mark.parametrize("rows", [2, 1])
def test_block_forward_fused_bc_fp16(rows):
    """An fp16 block (converted with .half(), no autocast) takes the fused path too,
    one workgroup per d at a batch of two and split halves at a batch of one: against
    the same block unfused and the CPU oracle of the block."""
    import mambaqc_amd

    torch.manual_seed(6)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=64).to(DEV, F16).eval()
    g = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(rows, 300, 64, generator=g, device=DEV).to(F16)
    assert blk._use_fused_bc(torch.empty(rows, 300, blk.d_inner, device=DEV, dtype=F16))
    print(f"fp16 block fused B{rows}", flush=True)
    with torch.no_grad():
        got = blk(x)
        blk.fuse_bc = False
        ref_unfused = blk(x)
        blk.fuse_bc = None
    assert got.dtype == F16
    assert_close(got, ref_unfused, 2e-2, "fp16 block fused vs unfused")
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.float().cpu(), d_state=64)
    assert_close(got, want, 2e-2, "fp16 block fused vs oracle")


@pytest.mark.parametrize("dt", [F16, BF], ids=["f16", "bf16"])
def test_block_forward_fused_bc_autocast(dt):
    """fp32 parameters in inference under autocast take the fused path, the
    projections' operands cast to autocast's dtype as F.linear's would be: against
    the same block with fusion off under the same autocast, and the CPU oracle of
    the block in fp32."""
    import mambaqc_amd

    torch.manual_seed(8)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=64).to(DEV).eval()
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(2, 300, 64, generator=g, device=DEV)
    print(f"autocast {dt} block fused", flush=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=dt):
        assert blk._use_fused_bc(torch.empty(2, 300, blk.d_inner, device=DEV, dtype=dt))
        got = blk(x)
        blk.fuse_bc = False
        ref_unfused = blk(x)
        blk.fuse_bc = None
    assert_close(got, ref_unfused, 2e-2, f"autocast {dt} block fused vs unfused")
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.cpu(), d_state=64)
    assert_close(got, want, 2e-2, f"autocast {dt} block fused vs oracle")
