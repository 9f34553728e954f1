"""GPU parity of the backward passes: HIP backward kernels (through their
torch.autograd.Function wrappers) against torch autograd through the CPU
oracle in float64 on the same (rounded) inputs. fp32 within rtol 1e-4,
bf16/fp16 within 2e-2, each with an atol floor of rtol * max|ref|.

The reference has no GPU backward at all (its Triton launches sit outside
autograd); the oracle's autograd is the only definition of these gradients.
"""
import pytest
import torch

import oracle
from conftest import assert_close, tol

import mambaqc_amd
from mambaqc_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _leaf(t, dev=None):
    t = t.detach()
    if dev is not None:
        t = t.to(dev)
    return t.requires_grad_(True)


def _dl_inputs(b, T, d, k, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    delta = torch.nn.functional.softplus(r(b, T, d) - 1).to(dtype)
    s = r(b, T, d).to(dtype)
    Bm = (r(b, T, d, k, 4) * 0.2).to(dtype)
    C = (r(b, T, d, k, 4) * 0.2).to(dtype)
    la = r(d, k) * 0.5 + 1
    li = r(d, k, 3) * 0.3
    D = torch.ones(d) + 0.1 * r(d)
    return [delta, s, Bm, C, la, li, D]


@pytest.mark.parametrize("shape", [(2, 37, 5, 16), (1, 20, 3, 5), (2, 9, 130, 64),
                                   (1, 1, 2, 1), (1, 50, 13, 32)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_dl_backward(shape, dtype):
    b, T, d, k = shape
    ins = _dl_inputs(b, T, d, k, seed=sum(shape), dtype=dtype)
    g = torch.Generator().manual_seed(7)
    gy = torch.randn(b, T, d, 4, generator=g).to(dtype)
    gh = torch.randn(b, d, k, 4, generator=g).to(dtype)
    h0 = (torch.randn(b, d, k, 4, generator=g) * 0.5).to(dtype)

    got_in = [_leaf(t, DEV) for t in ins] + [_leaf(h0, DEV)]
    y, hl = K.ssm_forward_fused_dl(*got_in[:7], h0=got_in[7], return_state=True)
    ((y.float() * gy.to(DEV).float()).sum() + (hl.float() * gh.to(DEV).float()).sum()).backward()

    ref_in = [_leaf(t.double()) for t in ins] + [_leaf(h0.double())]
    yr, hr = oracle.ssm_forward_dl_reference(*ref_in[:7], h0=ref_in[7], return_state=True)
    ((yr * gy.double()).sum() + (hr * gh.double()).sum()).backward()

    assert_close(y, yr, tol(dtype), f"y {shape} {dtype}")
    names = ["d_delta", "d_s", "dB", "dC", "dLambda_alpha", "dLambda_imag", "dD", "dh0"]
    for name, a, r in zip(names, got_in, ref_in):
        assert a.grad is not None, name
        assert a.grad.dtype == a.dtype, name
        assert_close(a.grad, r.grad, tol(dtype), f"{name} {shape} {dtype}")


@pytest.mark.parametrize("shape", [(2, 37, 5, 16), (1, 9, 13, 3), (2, 16, 8, 64)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_front_backward(shape, dtype):
    """Front (delta = softplus(dt_raw), s = sigmoid(g_raw) * x) + SSM as one
    autograd node, against torch autograd of the same composition on the
    oracle in float64. dt_raw has entries above softplus' threshold (20)."""
    b, T, d, k = shape
    ins = _dl_inputs(b, T, d, k, seed=sum(shape) + 1, dtype=dtype)
    g = torch.Generator().manual_seed(11)
    dt = (torch.randn(b, T, d, generator=g) - 1).to(dtype)
    dt[0, 0, 0] = 22.0
    gr = (torch.randn(b, T, d, generator=g) * 2).to(dtype)
    x = torch.randn(b, T, d, generator=g).to(dtype)
    gy = torch.randn(b, T, d, 4, generator=g).to(dtype)
    h0 = (torch.randn(b, d, k, 4, generator=g) * 0.5).to(dtype)
    rest = ins[2:]

    got_in = [_leaf(t, DEV) for t in [dt, gr, x] + rest + [h0]]
    y = K.ssm_forward_front_dl(*got_in[:8], h0=got_in[8])
    (y.float() * gy.to(DEV).float()).sum().backward()

    ref_in = [_leaf(t.double()) for t in [dt, gr, x] + rest + [h0]]
    delta = torch.nn.functional.softplus(ref_in[0])
    s = torch.sigmoid(ref_in[1]) * ref_in[2]
    yr = oracle.ssm_forward_dl_reference(delta, s, *ref_in[3:8], h0=ref_in[8])
    (yr * gy.double()).sum().backward()

    assert_close(y, yr, tol(dtype), f"y {shape} {dtype}")
    names = ["d_dt_raw", "d_g_raw", "d_x", "dB", "dC", "dLambda_alpha", "dLambda_imag", "dD",
             "dh0"]
    for name, a, r in zip(names, got_in, ref_in):
        assert a.grad is not None, name
        assert a.grad.dtype == a.dtype, name
        assert_close(a.grad, r.grad, tol(dtype), f"{name} {shape} {dtype}")


def test_ssm_dl_backward_without_state_terms():
    """No h0 and no gradient on the final state; some steps with a large delta
    (|q| close to 1 - 2/(1 + delta |a|/2)... i.e. strong damping)."""
    ins = _dl_inputs(2, 19, 4, 8, seed=3, dtype=torch.float32)
    ins[0][0, 3] = 40.0
    got_in = [_leaf(t, DEV) for t in ins]
    gy = torch.randn(2, 19, 4, 4, generator=torch.Generator().manual_seed(1))
    (K.ssm_forward_fused_dl(*got_in).float() * gy.to(DEV)).sum().backward()
    ref_in = [_leaf(t.double()) for t in ins]
    (oracle.ssm_forward_dl_reference(*ref_in) * gy.double()).sum().backward()
    for a, r, name in zip(got_in, ref_in, ["delta", "s", "B", "C", "la", "li", "D"]):
        assert_close(a.grad, r.grad, 1e-4, name)


@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_dl_backward_clamp_engaged(dtype):
    """Steps where the Cayley denominator's squared norm N falls below eps, so
    q = conj(den) (x) num / eps with N held constant (the reference's
    clamp_min). A large eps keeps those steps well conditioned; negative deltas
    at two steps put most lanes below it there while the other steps and
    chunks stay above."""
    b, T, d, k = 2, 11, 6, 8
    eps = 0.5
    ins = _dl_inputs(b, T, d, k, seed=5, dtype=dtype)
    ins[0][:, 3] = -1.6
    ins[0][1, 7] = -1.2
    # The clamp must engage at those steps for some lanes and not for others.
    a = -torch.nn.functional.softplus(ins[4].double())
    v = torch.tanh(ins[5].double())
    dl = ins[0].double()[..., None]
    N = 1 - dl * a + dl ** 2 * (a ** 2 + (v ** 2).sum(-1)) / 4
    assert (N[:, 3] < eps).any() and (N[:, 3] > eps).any()
    assert (N[:, :3] > eps).all() and (N[0, 4:] > eps).all()
    g = torch.Generator().manual_seed(9)
    gy = torch.randn(b, T, d, 4, generator=g).to(dtype)

    got_in = [_leaf(t, DEV) for t in ins]
    y = K.ssm_forward_fused_dl(*got_in, eps=eps)
    (y.float() * gy.to(DEV).float()).sum().backward()
    ref_in = [_leaf(t.double()) for t in ins]
    yr = oracle.ssm_forward_dl_reference(*ref_in, eps=eps)
    (yr * gy.double()).sum().backward()

    assert_close(y, yr, tol(dtype), f"y {dtype}")
    for a_, r_, name in zip(got_in, ref_in, ["delta", "s", "B", "C", "la", "li", "D"]):
        assert_close(a_.grad, r_.grad, tol(dtype), f"{name} {dtype}")


def test_ssm_dl_backward_config3_slices():
    """Config-3 sizes in bf16 (B4 T2048 D1536 S64): lanes are independent, so the
    per-(b, t, d) gradients of d-slices are checked against the oracle on the
    slice's own inputs; every lane is checked through linearity of the backward
    in gy (2 gy gives exactly twice every gradient up to rounding)."""
    b, T, d, k = 4, 2048, 1536, 64
    g = torch.Generator(device=DEV).manual_seed(0)
    bf = torch.bfloat16
    delta = torch.nn.functional.softplus(torch.randn(b, T, d, generator=g, device=DEV) - 2).to(bf)
    s = torch.randn(b, T, d, generator=g, device=DEV).to(bf)
    Bm = torch.randn(b, T, d, k, 4, generator=g, device=DEV, dtype=bf) * 0.02
    C = torch.randn(b, T, d, k, 4, generator=g, device=DEV, dtype=bf) * 0.02
    la = torch.randn(d, k, generator=g, device=DEV) * 0.5 + 1
    li = torch.randn(d, k, 3, generator=g, device=DEV) * 0.1
    D = torch.ones(d, device=DEV)
    gy = torch.randn(b, T, d, 4, generator=g, device=DEV).to(bf)
    leaves = [_leaf(t) for t in (delta, s, Bm, C, la, li, D)]
    y = K.ssm_forward_fused_dl(*leaves)
    grads = torch.autograd.grad(y, leaves, gy)
    grads2 = torch.autograd.grad(K.ssm_forward_fused_dl(*leaves), leaves, (2 * gy.float()).to(bf))
    for name, g1, g2 in zip(["delta", "s", "B", "C", "la", "li", "D"], grads, grads2):
        assert torch.isfinite(g1).all(), name
        assert_close(g2.float(), 2 * g1.float(), 2e-2, f"linearity {name}")
    del grads2
    # Both ends and the middle of the grid, in every batch row.
    for b0, ds in ((0, slice(0, 2)), (1, slice(380, 382)), (2, slice(766, 768)),
                   (3, slice(1150, 1152)), (3, slice(1534, 1536))):
        sl = [t[b0:b0 + 1, :, ds].detach().cpu().double() for t in (delta, s, Bm, C)]
        ref = [_leaf(t) for t in sl] + [_leaf(t[ds].detach().cpu().double()) for t in (la, li, D)]
        yr = oracle.ssm_forward_dl_reference(*ref)
        (yr * gy[b0:b0 + 1, :, ds].cpu().double()).sum().backward()
        for name, gg, r in zip(["delta", "s", "B", "C"], grads[:4], ref[:4]):
            assert_close(gg[b0:b0 + 1, :, ds], r.grad, 2e-2, f"C3 {name} b={b0} d={ds}")


@pytest.mark.parametrize("dm", [7, 64, 1536, 2100])
@pytest.mark.parametrize("dtype", DTYPES)
def test_qln_backward(dm, dtype):
    g = torch.Generator().manual_seed(dm)
    q = torch.randn(2, 3, dm, 4, generator=g).to(dtype)
    q[0, 1, : dm // 2] *= 1e-3            # small norms: the eps terms matter
    gamma = torch.rand(dm, generator=g) + 0.5
    beta = torch.randn(dm, 4, generator=g) * 0.1
    dout = torch.randn(2, 3, dm, 4, generator=g).to(dtype)
    a = [_leaf(t, DEV) for t in (q, gamma, beta)]
    (K.quaternion_layer_norm_fused(*a).float() * dout.to(DEV).float()).sum().backward()
    r = [_leaf(t.double()) for t in (q, gamma, beta)]
    (oracle.qln_reference(*r) * dout.double()).sum().backward()
    for name, x, y in zip(["dq", "dgamma", "dbeta"], a, r):
        assert_close(x.grad, y.grad, tol(dtype), f"qln {name} d={dm} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_out_gate_backward(dtype):
    rows, dm, di = 37, 24, 48
    g = torch.Generator().manual_seed(9)
    x = torch.randn(rows, dm, generator=g).to(dtype)
    xz = torch.randn(rows, 2 * di, generator=g).to(dtype)
    yr = torch.randn(rows, dm, generator=g).to(dtype)
    go = torch.randn(rows, dm, generator=g).to(dtype)
    xg, xzg, yg = (_leaf(t, DEV) for t in (x, xz, yr))
    z = xzg.chunk(2, dim=-1)[1]
    (mambaqc_amd.out_gate(xg, z, yg).float() * go.to(DEV).float()).sum().backward()
    xr, xzr, yrr = (_leaf(t.double()) for t in (x, xz, yr))
    zr = xzr.chunk(2, dim=-1)[1]
    ((xr + torch.sigmoid(zr[:, :dm]) * yrr) * go.double()).sum().backward()
    assert_close(xg.grad, xr.grad, tol(dtype), "dx")
    assert_close(xzg.grad, xzr.grad, tol(dtype), "dxz")
    assert_close(yg.grad, yrr.grad, tol(dtype), "dy")


def _block_grads_vs_oracle(d_model, d_state, expand, x_shape, seed):
    torch.manual_seed(seed)
    blk = mambaqc_amd.QuaternionMamba2Block(d_model, d_state=d_state, d_conv=4,
                                            expand_factor=expand)
    x = torch.randn(*x_shape)
    gout = torch.randn(*x_shape)
    sd = {k: _leaf(v.double()) for k, v in blk.state_dict().items()}
    xr = _leaf(x.double())
    (oracle.block_forward_reference(sd, xr, d_state=d_state) * gout.double()).sum().backward()
    blk = blk.to(DEV)
    xg = _leaf(x, DEV)
    (blk(xg) * gout.to(DEV)).sum().backward()
    assert_close(xg.grad, xr.grad, 1e-4, "block dx")
    for name, p in blk.named_parameters():
        assert p.grad is not None, name
        assert_close(p.grad, sd[name].grad, 1e-4, f"block d{name}")


def test_block_backward_config1():
    _block_grads_vs_oracle(64, 16, 2, (1, 64, 64), seed=0)


def test_block_backward_ragged():
    _block_grads_vs_oracle(24, 5, 2, (2, 19, 24), seed=4)


def test_block_backward_headline_width():
    """The headline configuration's width (d_model 768, d_state 64, expand 2:
    two 604 M-parameter projections) at B1 T32: every gradient of the block
    against fp64 autograd through the oracle."""
    _block_grads_vs_oracle(768, 64, 2, (1, 32, 768), seed=21)


def test_block_backward_chunked_walks():
    """Batch 1, 300 steps, 4 x 16 states: the SSM's training walk and backward
    run in time chunks (train_chunk_len < seq_len), inside the block's autograd."""
    from mambaqc_amd.kernels.ssm_fused import train_chunk_len
    assert train_chunk_len(1, 300, 64, 16, torch.float32) < 300
    _block_grads_vs_oracle(32, 16, 2, (1, 300, 32), seed=12)


def test_block_forward_backward_config4_fp16_autocast():
    """Config 4 at full size: B4 T2048 d768 s64, fp16 autocast, forward +
    backward of the whole block, with loss scaling as torch's GradScaler does it
    (the reference trainer uses one, train.py): the largest of 2^24, 2^20, 2^16
    whose gradients are all finite. Unscaled, fp16 gradients of a mean over
    6.3M outputs underflow in the torch GEMM backward (dt_proj). Every gradient
    is finite, non-zero, and within 5 % (relative Frobenius norm) of the same
    block's fp32 gradients, which the small-size tests pin to the oracle."""
    torch.manual_seed(0)
    blk = mambaqc_amd.QuaternionMamba2Block(768, d_state=64, d_conv=4, expand_factor=2).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(4, 2048, 768, generator=g, device=DEV)
    g16 = None
    for scale in (2.0 ** 24, 2.0 ** 20, 2.0 ** 16):
        blk.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            out = blk(x)
            loss = out.float().pow(2).mean()
        # fp32 residual stream + fp16 gate/projection promotes to fp32, as in the reference.
        assert out.dtype == torch.float32 and torch.isfinite(out).all()
        (loss * scale).backward()
        grads = {n: p.grad.detach().float() / scale for n, p in blk.named_parameters()}
        del out, loss
        if all(torch.isfinite(v).all() for v in grads.values()):
            g16 = grads
            break
    assert g16 is not None, "no loss scale gave finite fp16 gradients"
    blk.zero_grad(set_to_none=True)
    blk(x).pow(2).mean().backward()
    for n, p in blk.named_parameters():
        a, r = g16[n], p.grad.detach()
        assert a.abs().sum() > 0, n
        rel = ((a - r).norm() / r.norm()).item()
        assert rel < 5e-2, f"config 4 d{n}: fp16-autocast vs fp32 relative error {rel:.3g}"


def _close_on_device(got, ref, rtol, what):
    """assert_close's bound (rtol * |ref| + rtol * max|ref|) evaluated on the
    GPU in fp32, for gradients too large to copy to the host as float64."""
    got = got.float()
    ref = ref.float()
    assert got.shape == ref.shape, what
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    scale = ref.abs().max()
    excess = (got - ref).abs() - rtol * (ref.abs() + scale)
    worst = int(torch.argmax(excess))
    assert excess.reshape(-1)[worst] <= 0, (
        f"{what}: {int((excess > 0).sum())}/{ref.numel()} out of rtol {rtol}; worst at "
        f"{worst}: got {got.reshape(-1)[worst].item():.6g}, ref {ref.reshape(-1)[worst].item():.6g}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_linear_backward_at_projection_shape(dtype):
    """The B/C projections' blocked GEMMs at the shape config 4 trains them:
    K 1536 inputs, N 393 216 outputs (d_inner 1536 x d_state 64 x 4), here
    1024 token rows (the blocked path's threshold). The forward by column
    blocks, dX as one batched GEMM over equal K blocks with fp32 partials, dW
    by row blocks, against one unblocked F.linear with autograd in fp32 on the
    same rounded operands (torch's GEMM as the third-party reference)."""
    from mambaqc_amd.layers import quaternion_linear as ql

    m, k, n = 1024, 1536, 393216
    print(f"wide_linear backward {dtype} M{m} K{k} N{n}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(m, k, generator=g, device=DEV).to(dtype)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(dtype)
    gy = torch.randn(m, n, generator=g, device=DEV).to(dtype)
    es = w.element_size()
    assert len(ql._blocks(n, k, es)) > 1 and ql._dx_batches(n, k, es) >= 8
    assert m >= ql.WIDE_LINEAR_MIN_ROWS
    xb, wb = _leaf(x), _leaf(w)
    y = ql.wide_linear(xb, wb)
    assert isinstance(y.grad_fn, torch.autograd.function.BackwardCFunction)
    y.backward(gy)
    xf, wf = _leaf(x.float()), _leaf(w.float())
    yf = torch.nn.functional.linear(xf, wf)
    yf.backward(gy.float())
    _close_on_device(y, yf, 2e-2, f"wide_linear y {dtype}")
    _close_on_device(xb.grad, xf.grad, 2e-2, f"wide_linear dX {dtype}")
    _close_on_device(wb.grad, wf.grad, 2e-2, f"wide_linear dW {dtype}")


@pytest.mark.parametrize("shape", [(2, 37, 48, 4), (1, 3, 16, 4), (2, 20, 13, 3), (3, 33, 64, 6)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_causal_conv_silu_backward(shape, dtype):
    from mambaqc_amd.layers.causal_conv1d import causal_conv1d_silu
    b, T, C, K = shape
    g = torch.Generator().manual_seed(sum(shape) + 1)
    xz = torch.randn(b, T, 2 * C, generator=g).to(dtype)
    w = torch.randn(C, 1, K, generator=g) * 0.5
    bias = torch.randn(C, generator=g) * 0.1
    gout = torch.randn(b, T, C, generator=g).to(dtype)
    xzg, wg, bg = _leaf(xz, DEV), _leaf(w, DEV), _leaf(bias, DEV)
    out = causal_conv1d_silu(xzg.chunk(2, dim=-1)[0], wg, bg)
    (out.float() * gout.to(DEV).float()).sum().backward()
    xzr, wr, br = _leaf(xz.double()), _leaf(w.double()), _leaf(bias.double())
    xt = torch.nn.functional.pad(xzr[..., :C].transpose(1, 2), (K - 1, 0))
    ref = torch.nn.functional.silu(torch.nn.functional.conv1d(xt, wr, br, groups=C)).transpose(1, 2)
    (ref * gout.double()).sum().backward()
    assert_close(xzg.grad, xzr.grad, tol(dtype), f"dx {shape} {dtype}")
    assert_close(wg.grad, wr.grad, tol(dtype), f"dw {shape} {dtype}")
    assert_close(bg.grad, br.grad, tol(dtype), f"dbias {shape} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_empty_sequence(dtype):
    """seq_len 0: y is empty, the final state is h0 (zeros without h0), and the
    backward passes dL/dh_last straight to h0 with zero parameter gradients."""
    b, d, k = 2, 5, 16
    ins = _dl_inputs(b, 0, d, k, seed=1, dtype=dtype)
    g = torch.Generator().manual_seed(2)
    h0 = torch.randn(b, d, k, 4, generator=g).to(dtype)
    gh = torch.randn(b, d, k, 4, generator=g).to(dtype)

    y, hl = K.ssm_forward_fused_dl(*(t.to(DEV) for t in ins), h0=h0.to(DEV), return_state=True)
    assert y.shape == (b, 0, d, 4)
    assert hl.dtype == torch.float32  # the state is fp32 at every storage dtype
    assert torch.equal(hl.cpu(), h0.float())
    _, hl0 = K.ssm_forward_fused_dl(*(t.to(DEV) for t in ins), return_state=True)
    assert (hl0 == 0).all()

    got = [_leaf(t, DEV) for t in ins] + [_leaf(h0, DEV)]
    y, hl = K.ssm_forward_fused_dl(*got[:7], h0=got[7], return_state=True)
    (hl.float() * gh.to(DEV).float()).sum().backward()
    assert torch.equal(hl.detach().cpu(), h0.float())
    assert torch.equal(got[7].grad.cpu(), gh)
    for t, name in zip(got[4:7], ["lambda_alpha", "lambda_imag", "D"]):
        assert t.grad is not None and (t.grad == 0).all(), name


def test_training_after_inference_mode():
    """A bf16 block run under torch.inference_mode, then trained: the library's
    fp32 copies of its small parameters, converted during inference mode, are
    ordinary tensors that the training step can save for its backward."""
    torch.manual_seed(8)
    blk = mambaqc_amd.QuaternionMamba2Block(32, d_state=8).to(DEV, torch.bfloat16)
    x = torch.randn(2, 30, 32, device=DEV).to(torch.bfloat16)
    with torch.inference_mode():
        y0 = blk(x)
    xr = x.clone().requires_grad_()
    y = blk(xr)
    y.float().pow(2).mean().backward()
    # (the training walk and the inference walk sum over d_state in different orders)
    assert_close(y, y0.clone(), 2e-2, "training forward after inference mode")
    assert xr.grad is not None and torch.isfinite(xr.grad.float()).all()
    assert all(p.grad is not None for p in blk.parameters())
