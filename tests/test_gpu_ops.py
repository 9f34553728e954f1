"""GPU tests of the registered operators (torch.ops.mambaqc.*): each equals the
Python API it wraps, torch.library.opcheck passes (schema, fake kernel against
the real one, autograd registration, AOT dispatch), gradients through the ops
equal those of the package's autograd Functions, and a torch.compile'd
(aot_eager) pipeline of ops equals the eager one."""
import pytest
import torch

import mambaqc_amd
from mambaqc_amd import kernels as K
from mambaqc_amd.block import out_gate as api_out_gate
from mambaqc_amd.layers.causal_conv1d import causal_conv1d_silu as api_conv

pytestmark = pytest.mark.gpu
DEV = "cuda"
mm = torch.ops.mambaqc


def _g(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _dl_inputs(b=2, t=37, d=6, n=8, dtype=torch.bfloat16, seed=0, grad=False):
    g = _g(seed)
    delta = torch.nn.functional.softplus(torch.randn(b, t, d, generator=g, device=DEV) - 1).to(dtype)
    s = torch.randn(b, t, d, generator=g, device=DEV).to(dtype)
    B = (torch.randn(b, t, d, n, 4, generator=g, device=DEV) * 0.3).to(dtype)
    C = (torch.randn(b, t, d, n, 4, generator=g, device=DEV) * 0.3).to(dtype)
    la = torch.randn(d, n, generator=g, device=DEV) * 0.5 + 1
    li = torch.randn(d, n, 3, generator=g, device=DEV) * 0.1
    D = torch.randn(d, generator=g, device=DEV)
    h0 = torch.randn(b, d, n, 4, generator=g, device=DEV) * 0.1
    ts = [delta, s, B, C, la, li, D, h0]
    if grad:
        ts = [x.detach().requires_grad_() for x in ts]
    return ts


def test_ops_equal_python_api():
    g = _g(1)
    p = torch.randn(3, 5, 4, generator=g, device=DEV)
    q = torch.randn(3, 5, 4, generator=g, device=DEV)
    assert torch.equal(mm.quaternion_multiply(p, q), K.quaternion_multiply(p, q))
    assert torch.equal(mm.quaternion_conjugate(p), K.quaternion_conjugate(p))
    assert torch.equal(mm.quaternion_inverse(p, 1e-6), K.quaternion_inverse(p, 1e-6))
    assert torch.equal(mm.quaternion_norm(p), K.quaternion_norm(p))
    z = torch.randn(2, 9, 3, 4, 4, generator=g, device=DEV) * 0.3
    assert torch.equal(mm.cayley_discretization(z, 1e-6), K.cayley_discretization_fused(z, 1e-6))
    qq = mm.cayley_discretization(z, 1e-6)
    assert torch.equal(mm.cumprod_scan(qq), K.parallel_scan_quaternion(qq))
    Bq = torch.randn(2, 9, 3, 4, 4, generator=g, device=DEV) * 0.3
    Cq = torch.randn(2, 9, 3, 4, 4, generator=g, device=DEV) * 0.3
    Sq = torch.randn(2, 9, 3, 4, generator=g, device=DEV)
    Dq = torch.randn(2, 9, 3, generator=g, device=DEV)
    assert torch.equal(mm.ssm_forward_q(qq, Bq, Sq, Cq, Dq), K.ssm_forward_fused(qq, Bq, Sq, Cq, Dq))
    h = torch.randn(2, 3, 4, 4, generator=g, device=DEV)
    got = mm.ssm_step_q(qq[:, 0], Bq[:, 0], Sq[:, 0], Cq[:, 0], Dq[:, 0], h)
    want = K.ssm_step_fused(qq[:, 0], Bq[:, 0], Sq[:, 0], Cq[:, 0], Dq[:, 0], h)
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    delta, s, B, C, la, li, D, h0 = _dl_inputs()
    for chunk_len in (None, 10):
        y, hl = mm.ssm_forward_dl(delta, s, B, C, la, li, D, h0, 1e-6, chunk_len)
        y2, hl2 = K.ssm_forward_fused_dl(delta, s, B, C, la, li, D, h0=h0, return_state=True,
                                         chunk_len=chunk_len)
        assert torch.equal(y, y2) and torch.equal(hl, hl2)
    yt, hlt, ck = mm.ssm_forward_dl_train(delta, s, B, C, la, li, D, h0)
    assert torch.equal(yt, mm.ssm_forward_dl(delta, s, B, C, la, li, D, h0)[0])
    assert ck.dtype == torch.float32 and ck.shape == (2, 5, 6, 8, 4)
    dt = torch.randn(2, 9, 6, generator=g, device=DEV)
    gr = torch.randn(2, 9, 6, generator=g, device=DEV)
    x = torch.randn(2, 9, 6, generator=g, device=DEV)
    assert all(torch.equal(a, b) for a, b in zip(mm.ssm_front(dt, gr, x), K.ssm_front(dt, gr, x)))
    yq = torch.randn(2, 9, 6, 4, generator=g, device=DEV)
    gam, bet = torch.rand(6, device=DEV) + 0.5, torch.randn(6, 4, device=DEV) * 0.1
    out, mean, rstd = mm.quaternion_layer_norm(yq, gam, bet, 1e-5)
    o2, m2, r2 = K.quaternion_layer_norm_fused(yq, gam, bet, 1e-5, return_stats=True)
    assert torch.equal(out, o2) and torch.equal(mean, m2) and torch.equal(rstd, r2)
    w, bias = torch.randn(6, 1, 4, generator=g, device=DEV), torch.randn(6, generator=g, device=DEV)
    with torch.no_grad():
        assert torch.equal(mm.causal_conv1d_silu(x, w, bias), api_conv(x, w, bias))
        xz = torch.randn(2, 9, 12, generator=g, device=DEV)
        yr = torch.randn(2, 9, 6, generator=g, device=DEV)
        assert torch.equal(mm.out_gate(x, xz[..., 6:], yr), api_out_gate(x, xz[..., 6:], yr))


def test_opcheck():
    """torch.library.opcheck on one case per op family (fp32, small)."""
    from torch.library import opcheck
    g = _g(2)
    p = torch.randn(3, 4, generator=g, device=DEV, requires_grad=True)
    q = torch.randn(3, 4, generator=g, device=DEV, requires_grad=True)
    opcheck(mm.quaternion_multiply, (p, q))
    opcheck(mm.quaternion_conjugate, (p,))
    opcheck(mm.quaternion_norm, (p.detach(),))
    z = torch.randn(2, 5, 3, 2, 4, generator=g, device=DEV) * 0.3
    opcheck(mm.cayley_discretization, (z, 1e-6))
    opcheck(mm.cumprod_scan, (z,))
    delta, s, B, C, la, li, D, h0 = _dl_inputs(dtype=torch.float32, t=13, grad=True)
    opcheck(mm.ssm_forward_dl_train, (delta, s, B, C, la, li, D, h0, 1e-6))
    dtr = torch.randn(delta.shape, generator=g, device=DEV, requires_grad=True)
    grr = torch.randn(delta.shape, generator=g, device=DEV, requires_grad=True)
    opcheck(mm.ssm_front_forward_dl_train, (dtr, grr, s, B, C, la, li, D, h0, 1e-6))
    with torch.no_grad():
        opcheck(mm.ssm_forward_dl, (delta, s, B, C, la, li, D, None, 1e-6, None))
    x = torch.randn(2, 7, 6, generator=g, device=DEV, requires_grad=True)
    opcheck(mm.ssm_front, (x, x.detach().clone().requires_grad_(), x.detach().clone()))
    yq = torch.randn(2, 7, 6, 4, generator=g, device=DEV, requires_grad=True)
    gam = (torch.rand(6, device=DEV) + 0.5).requires_grad_()
    bet = (torch.randn(6, 4, device=DEV) * 0.1).requires_grad_()
    opcheck(mm.quaternion_layer_norm, (yq, gam, bet, 1e-5))
    w = torch.randn(6, 1, 4, generator=g, device=DEV, requires_grad=True)
    bias = torch.randn(6, generator=g, device=DEV, requires_grad=True)
    opcheck(mm.causal_conv1d_silu, (x, w, bias))
    xz = torch.randn(2, 7, 12, generator=g, device=DEV, requires_grad=True)
    yr = torch.randn(2, 7, 6, generator=g, device=DEV, requires_grad=True)
    opcheck(mm.out_gate, (x, xz, yr))
    # The fused B/C walk (bf16, inference only).
    bf = torch.bfloat16
    xb = torch.randn(1, 9, 64, generator=g, device=DEV).to(bf)
    wb = (torch.randn(64 * 4 * 4, 64, generator=g, device=DEV) * 0.05).to(bf)
    wc = (torch.randn(64 * 4 * 4, 64, generator=g, device=DEV) * 0.05).to(bf)
    db = torch.nn.functional.softplus(torch.randn(1, 9, 64, generator=g, device=DEV)).to(bf)
    sb = torch.randn(1, 9, 64, generator=g, device=DEV).to(bf)
    lab = torch.randn(64, 4, generator=g, device=DEV) * 0.5 + 1
    lib_ = torch.randn(64, 4, 3, generator=g, device=DEV) * 0.1
    Db = torch.ones(64, device=DEV)
    with torch.no_grad():
        opcheck(mm.ssm_forward_fused_bc, (xb, wb, wc, db, sb, lab, lib_, Db, None, 1e-6))


def _grads(out, inputs, seed=5):
    gs = [torch.randn(o.shape, generator=_g(seed + i), device=DEV).to(o.dtype)
          for i, o in enumerate(out)]
    return torch.autograd.grad(out, [t for t in inputs if t is not None], gs, allow_unused=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ssm_train_op_gradients_equal_autograd_function(dtype):
    ins = _dl_inputs(dtype=dtype, grad=True)
    y, hl, _ = mm.ssm_forward_dl_train(*ins, 1e-6)
    got = _grads((y, hl), ins)
    ins2 = [t.detach().requires_grad_() for t in ins]
    y2, hl2 = K.ssm_forward_fused_dl(*ins2[:7], eps=1e-6, h0=ins2[7], return_state=True)
    want = _grads((y2, hl2), ins2)
    assert torch.equal(y, y2) and torch.equal(hl, hl2)
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"grad {i}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_front_train_op_gradients_equal_autograd_function(dtype):
    """The front + training-walk operator (what torch.compile traces while
    autograd records) against the eager _SsmFrontFusedDL: the same kernels in
    the same order, d_delta and d_s fp32 into the front's backward in both, so
    equal bit for bit (fp16 included, where a round trip through delta's dtype
    would not be)."""
    _, _, B, C, la, li, D, h0 = _dl_inputs(dtype=dtype, seed=3)
    g = _g(4)
    dt = torch.randn(B.shape[:3], generator=g, device=DEV).to(dtype)
    gr = torch.randn(B.shape[:3], generator=g, device=DEV).to(dtype)
    x = torch.randn(B.shape[:3], generator=g, device=DEV).to(dtype)
    ins = [t.detach().requires_grad_() for t in (dt, gr, x, B, C, la, li, D, h0)]
    y, hl, _ = mm.ssm_front_forward_dl_train(*ins, 1e-6)
    got = _grads((y, hl), ins)
    ins2 = [t.detach().requires_grad_() for t in ins]
    y2, hl2 = K.ssm_forward_front_dl(*ins2[:8], eps=1e-6, h0=ins2[8], return_state=True)
    want = _grads((y2, hl2), ins2)
    assert torch.equal(y, y2) and torch.equal(hl, hl2)
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"grad {i}"


def test_layer_ops_gradients_equal_autograd_functions():
    g = _g(7)
    yq = torch.randn(2, 7, 6, 4, generator=g, device=DEV, requires_grad=True)
    gam = (torch.rand(6, device=DEV) + 0.5).requires_grad_()
    bet = (torch.randn(6, 4, device=DEV) * 0.1).requires_grad_()
    out = mm.quaternion_layer_norm(yq, gam, bet, 1e-5)[0]
    ins2 = [t.detach().requires_grad_() for t in (yq, gam, bet)]
    out2 = K.quaternion_layer_norm_fused(*ins2, 1e-5)
    for a, b in zip(_grads((out,), (yq, gam, bet)), _grads((out2,), ins2)):
        assert torch.equal(a, b)
    x = torch.randn(2, 9, 6, generator=g, device=DEV, requires_grad=True)
    w = torch.randn(6, 1, 4, generator=g, device=DEV, requires_grad=True)
    bias = torch.randn(6, generator=g, device=DEV, requires_grad=True)
    ins2 = [t.detach().requires_grad_() for t in (x, w, bias)]
    for a, b in zip(_grads((mm.causal_conv1d_silu(x, w, bias),), (x, w, bias)),
                    _grads((api_conv(*ins2),), ins2)):
        assert torch.equal(a, b)
    xz = torch.randn(2, 9, 12, generator=g, device=DEV, requires_grad=True)
    yr = torch.randn(2, 9, 6, generator=g, device=DEV, requires_grad=True)
    ins2 = [t.detach().requires_grad_() for t in (x, xz, yr)]
    for a, b in zip(_grads((mm.out_gate(x, xz[..., 6:], yr),), (x, xz, yr)),
                    _grads((api_out_gate(ins2[0], ins2[1][..., 6:], ins2[2]),), ins2)):
        assert torch.equal(a, b)
    p = torch.randn(3, 4, generator=g, device=DEV, requires_grad=True)
    q = torch.randn(3, 4, generator=g, device=DEV, requires_grad=True)
    gp, gq = _grads((mm.quaternion_multiply(p, q),), (p, q))
    # Against torch autograd through the Hamilton product written out in torch.
    pr, qr = p.detach().double().requires_grad_(), q.detach().double().requires_grad_()
    w1, x1, y1, z1 = pr.unbind(-1)
    w2, x2, y2, z2 = qr.unbind(-1)
    ref = torch.stack([w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2, w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                       w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2, w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2], -1)
    rp, rq = _grads((ref,), (pr, qr))
    assert torch.allclose(gp.double(), rp, atol=1e-5) and torch.allclose(gq.double(), rq, atol=1e-5)


def test_compiled_pipeline_equals_eager():
    """front -> SSM -> QLN -> gate as ops under torch.compile (aot_eager: the
    graph is traced through the fake kernels, the ops run as themselves)."""
    blk = mambaqc_amd.QuaternionMamba2Block(32, d_state=8).to(DEV)
    g = _g(9)
    b, t, d, n = 2, 40, 64, 8
    xa = torch.randn(b, t, d, generator=g, device=DEV)
    dt = torch.randn(b, t, d, generator=g, device=DEV)
    gr = torch.randn(b, t, d, generator=g, device=DEV)
    Bq = torch.randn(b, t, d, n, 4, generator=g, device=DEV) * 0.2
    Cq = torch.randn(b, t, d, n, 4, generator=g, device=DEV) * 0.2
    x = torch.randn(b, t, 32, generator=g, device=DEV)
    z = torch.randn(b, t, d, generator=g, device=DEV)

    def pipeline(xa, dt, gr, Bq, Cq, x, z, yproj):
        delta, s = mm.ssm_front(dt, gr, xa)
        y, _ = mm.ssm_forward_dl(delta, s, Bq, Cq, blk.Lambda_alpha, blk.Lambda_imag, blk.D,
                                 None, 1e-6, None)
        yn, _, _ = mm.quaternion_layer_norm(y, blk.norm.gamma, blk.norm.beta, 1e-5)
        return mm.out_gate(x, z, yn.reshape(b, t, d * 4) @ yproj)

    yproj = torch.randn(d * 4, 32, generator=g, device=DEV) * 0.05
    with torch.no_grad():
        want = pipeline(xa, dt, gr, Bq, Cq, x, z, yproj)
        fn = torch.compile(pipeline, backend="aot_eager", fullgraph=True)
        got = fn(xa, dt, gr, Bq, Cq, x, z, yproj)
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype,rtol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_block_compiles_fullgraph(dtype, rtol):
    """torch.compile(block, fullgraph=True) traces the whole block: the kernels
    enter the graph as torch.ops.mambaqc.* operators. Forward and gradients
    against the eager block (aot_eager runs the traced graph as is)."""
    torch.manual_seed(3)
    blk = mambaqc_amd.QuaternionMamba2Block(32, d_state=8).to(DEV, dtype)
    x = torch.randn(2, 40, 32, generator=_g(4), device=DEV).to(dtype)
    compiled = torch.compile(blk, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        want = blk(x)
        got = compiled(x)
    from conftest import assert_close
    assert_close(got, want, rtol, "compiled block forward (no grad)")
    xe = x.clone().requires_grad_()
    xc = x.clone().requires_grad_()
    gy = torch.randn(want.shape, generator=_g(5), device=DEV).to(dtype)
    ye = blk(xe)
    ge = torch.autograd.grad(ye, [xe] + list(blk.parameters()), gy)
    yc = compiled(xc)
    gc = torch.autograd.grad(yc, [xc] + list(blk.parameters()), gy)
    assert_close(yc, ye, rtol, "compiled block forward (training)")
    names = ["x"] + [n for n, _ in blk.named_parameters()]
    for n, a, b in zip(names, gc, ge):
        assert_close(a, b, max(rtol, 1e-4), f"compiled block grad {n}")


def test_block_compiles_fullgraph_fp16_autocast():
    """The compiled block under fp16 autocast (config 4's precision): forward
    and gradients against the eager block. The traced front + SSM is one
    operator, so d_delta and d_s reach the front's backward in fp32 as in the
    eager path."""
    torch.manual_seed(5)
    blk = mambaqc_amd.QuaternionMamba2Block(32, d_state=8).to(DEV)
    x = torch.randn(2, 40, 32, generator=_g(6), device=DEV)
    compiled = torch.compile(blk, backend="aot_eager", fullgraph=True)
    gy = torch.randn(2, 40, 32, generator=_g(7), device=DEV)
    xe = x.clone().requires_grad_()
    xc = x.clone().requires_grad_()
    from conftest import assert_close
    with torch.autocast("cuda", dtype=torch.float16):
        ye = blk(xe)
        yc = compiled(xc)
    ge = torch.autograd.grad(ye.float(), [xe] + list(blk.parameters()), gy)
    gc = torch.autograd.grad(yc.float(), [xc] + list(blk.parameters()), gy)
    assert_close(yc, ye, 2e-2, "compiled block forward (fp16 autocast)")
    names = ["x"] + [n for n, _ in blk.named_parameters()]
    for n, a, b in zip(names, gc, ge):
        assert_close(a, b, 2e-2, f"compiled block grad {n} (fp16 autocast)")


def test_block_compiles_fused_bc_inference():
    """A compiled bf16 block in inference takes the fused B/C walk as the operator
    torch.ops.mambaqc.ssm_forward_fused_bc (sequences of FUSED_BC_MIN_SEQ tokens and
    more): its output against the eager block, which runs the same kernel, and
    against the compiled block with fusion off."""
    from mambaqc_amd.block import FUSED_BC_MIN_SEQ
    from conftest import assert_close

    torch.manual_seed(6)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16).to(DEV, torch.bfloat16).eval()
    x = torch.randn(2, FUSED_BC_MIN_SEQ + 44, 64, generator=_g(8), device=DEV).to(torch.bfloat16)
    compiled = torch.compile(blk, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        want = blk(x)
        got = compiled(x)
        blk.fuse_bc = False
        torch._dynamo.reset()
        unfused = torch.compile(blk, backend="aot_eager", fullgraph=True)(x)
        blk.fuse_bc = None
    assert torch.equal(got, want)
    assert_close(got, unfused, 2e-2, "compiled block, fused vs unfused B/C")
