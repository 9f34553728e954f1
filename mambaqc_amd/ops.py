"""torch.ops.mambaqc.*: the library's HIP kernels as registered PyTorch operators.

The reference calls its kernels as Python functions (mambaqc/kernels/__init__.py:10-33),
which this package mirrors in `mambaqc_amd.kernels`. This module registers the
same kernels with torch.library as custom operators, each with:
  - its implementation: the package's Python API (one launch through
    libmambaqc_hip.so on the tensors' device and current stream);
  - a fake implementation: output shapes and dtypes without running anything,
    so torch.compile / torch.export can trace graphs that call the ops and
    FakeTensorMode / the meta device can run them;
  - for the ops on the training path, an autograd formula made of the
    library's HIP backward kernels (registered as ops of their own).

Ops whose reference function has no gradient (Cayley, the cumulative product,
inverse, norm, the q-form SSM) register none, as in the reference.
`ssm_forward_dl` is the inference walk (whole or time-chunked); gradients go
through `ssm_forward_dl_train`, which also returns the fp32 state checkpoints
its backward reads. Optional tensor outputs are returned as empty tensors
(numel 0) where they do not apply.
"""
from typing import Optional, Tuple

import torch
from torch.library import custom_op, register_autograd

from . import _native as nat
from .block import _gate_operands, _out_gate_backward
from .kernels import cayley_transform, parallel_scan, quaternion_ops
from .kernels import ssm_fused as sf
from .kernels.quaternion_norm import _qln_backward, _qln_forward
from .layers.causal_conv1d import _conv_silu_backward, _ConvSiLU, _rows_view

NS = "mambaqc"
Tensor = torch.Tensor


# --- quaternion element-wise ops (reference quaternion_ops.py:259-461) --------

@custom_op(f"{NS}::quaternion_multiply", mutates_args=())
def quaternion_multiply(p: Tensor, q: Tensor) -> Tensor:
    return quaternion_ops.quaternion_multiply(p, q)


@quaternion_multiply.register_fake
def _(p, q):
    torch._check(p.shape == q.shape and p.shape[-1] == 4, lambda: "quaternion_multiply shapes")
    return torch.empty_like(p, memory_format=torch.contiguous_format)


def _qmul_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _qmul_backward(ctx, g):
    # <p (x) q, g> = <p, g (x) conj(q)> = <q, conj(p) (x) g> for real inner products.
    p, q = ctx.saved_tensors
    g = g.contiguous()
    gp = gq = None
    if ctx.needs_input_grad[0]:
        gp = quaternion_multiply(g, quaternion_conjugate(q))
    if ctx.needs_input_grad[1]:
        gq = quaternion_multiply(quaternion_conjugate(p), g)
    return gp, gq


@custom_op(f"{NS}::quaternion_conjugate", mutates_args=())
def quaternion_conjugate(q: Tensor) -> Tensor:
    return quaternion_ops.quaternion_conjugate(q)


@quaternion_conjugate.register_fake
def _(q):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


register_autograd(f"{NS}::quaternion_multiply", _qmul_backward, setup_context=_qmul_setup)
register_autograd(f"{NS}::quaternion_conjugate",
                  lambda ctx, g: quaternion_conjugate(g.contiguous()))


@custom_op(f"{NS}::quaternion_inverse", mutates_args=())
def quaternion_inverse(q: Tensor, eps: float = 1e-6) -> Tensor:
    return quaternion_ops.quaternion_inverse(q, eps)


@quaternion_inverse.register_fake
def _(q, eps=1e-6):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@custom_op(f"{NS}::quaternion_norm", mutates_args=())
def quaternion_norm(q: Tensor) -> Tensor:
    return quaternion_ops.quaternion_norm(q)


@quaternion_norm.register_fake
def _(q):
    return q.new_empty(q.shape[:-1])


# --- Cayley and the cumulative product (cayley_transform.py:199-223,
#     parallel_scan.py:171-295) -------------------------------------------------

@custom_op(f"{NS}::cayley_discretization", mutates_args=())
def cayley_discretization(z: Tensor, eps: float = 1e-6) -> Tensor:
    return cayley_transform.cayley_discretization_fused(z, eps)


@cayley_discretization.register_fake
def _(z, eps=1e-6):
    return torch.empty_like(z, memory_format=torch.contiguous_format)


@custom_op(f"{NS}::cumprod_scan", mutates_args=())
def cumprod_scan(q: Tensor) -> Tensor:
    return parallel_scan.parallel_scan_quaternion(q)


@cumprod_scan.register_fake
def _(q):
    torch._check(q.dim() == 5 and q.shape[-1] == 4, lambda: "cumprod_scan: [B, T, D, S, 4]")
    return torch.empty_like(q, memory_format=torch.contiguous_format)


# --- the q-form SSM (ssm_fused.py:258-401) -------------------------------------

@custom_op(f"{NS}::ssm_forward_q", mutates_args=())
def ssm_forward_q(q: Tensor, B: Tensor, S: Tensor, C: Tensor, D: Tensor) -> Tensor:
    return sf.ssm_forward_fused(q, B, S, C, D)


@ssm_forward_q.register_fake
def _(q, B, S, C, D):
    b, t, d, _, _ = q.shape
    return q.new_empty(b, t, d, 4)


@custom_op(f"{NS}::ssm_step_q", mutates_args=())
def ssm_step_q(q: Tensor, B: Tensor, S: Tensor, C: Tensor, D: Tensor,
               h_prev: Tensor) -> Tuple[Tensor, Tensor]:
    return sf.ssm_step_fused(q, B, S, C, D, h_prev)


@ssm_step_q.register_fake
def _(q, B, S, C, D, h_prev):
    b, d, n, _ = q.shape
    return q.new_empty(b, d, n, 4), q.new_empty(b, d, 4)


# --- the block's SSM, delta/Lambda form (quaternion_mamba2_block.py:168-230) ---

@custom_op(f"{NS}::ssm_forward_dl", mutates_args=())
def ssm_forward_dl(delta: Tensor, s: Tensor, B: Tensor, C: Tensor, lambda_alpha: Tensor,
                   lambda_imag: Tensor, D: Tensor, h0: Optional[Tensor] = None,
                   eps: float = 1e-6, chunk_len: Optional[int] = None) -> Tuple[Tensor, Tensor]:
    """Inference walk: (y [B, T, D, 4] in B's dtype, h_last [B, D, S, 4] fp32)."""
    with torch.no_grad():
        return sf.ssm_forward_fused_dl(delta, s, B, C, lambda_alpha, lambda_imag, D, eps=eps,
                                       h0=h0, return_state=True, chunk_len=chunk_len)


@ssm_forward_dl.register_fake
def _(delta, s, B, C, lambda_alpha, lambda_imag, D, h0=None, eps=1e-6, chunk_len=None):
    b, t, d, n, _ = B.shape
    return B.new_empty(b, t, d, 4), B.new_empty(b, d, n, 4, dtype=torch.float32)


@custom_op(f"{NS}::ssm_forward_fused_bc", mutates_args=())
def ssm_forward_fused_bc(x: Tensor, B_weight: Tensor, C_weight: Tensor, delta: Tensor, s: Tensor,
                         lambda_alpha: Tensor, lambda_imag: Tensor, D: Tensor,
                         h0: Optional[Tensor] = None,
                         eps: float = 1e-6) -> Tuple[Tensor, Tensor]:
    """The B/C projections and the inference walk in one kernel (bf16 or fp16):
    (y [B, T, D, 4] in x's dtype, h_last [B, D, S, 4] fp32). Inference only."""
    with torch.no_grad():
        return sf.ssm_forward_fused_bc(x, B_weight, C_weight, delta, s, lambda_alpha, lambda_imag,
                                       D, eps=eps, h0=h0, return_state=True)


@ssm_forward_fused_bc.register_fake
def _(x, B_weight, C_weight, delta, s, lambda_alpha, lambda_imag, D, h0=None, eps=1e-6):
    b, t, d = x.shape
    return (x.new_empty(b, t, d, 4), x.new_empty(b, d, lambda_alpha.shape[-1], 4,
                                                 dtype=torch.float32))


@custom_op(f"{NS}::ssm_forward_dl_train", mutates_args=())
def ssm_forward_dl_train(delta: Tensor, s: Tensor, B: Tensor, C: Tensor, lambda_alpha: Tensor,
                         lambda_imag: Tensor, D: Tensor, h0: Optional[Tensor] = None,
                         eps: float = 1e-6) -> Tuple[Tensor, Tensor, Tensor]:
    """Training walk: (y, h_last fp32, fp32 state checkpoints for the backward)."""
    y, h_last, saved = sf.ssm_fused_dl_train_forward(delta, s, B, C, lambda_alpha,
                                                     lambda_imag, D, h0, eps)
    return y, h_last, saved[-1]


def _ckpt_shape(B: Tensor):
    b, t, d, n, _ = B.shape
    every = int(nat.load().mqc_ssm_bwd_ckpt_every(nat.dtype_code(B)))
    return b, torch.sym_max((t + every - 1) // every, 1), d, n, 4


@ssm_forward_dl_train.register_fake
def _(delta, s, B, C, lambda_alpha, lambda_imag, D, h0=None, eps=1e-6):
    b, t, d, n, _ = B.shape
    return (B.new_empty(b, t, d, 4), B.new_empty(b, d, n, 4, dtype=torch.float32),
            B.new_empty(*_ckpt_shape(B), dtype=torch.float32))


@custom_op(f"{NS}::ssm_backward_dl", mutates_args=())
def ssm_backward_dl(delta: Tensor, s: Tensor, B: Tensor, C: Tensor, lambda_alpha: Tensor,
                    lambda_imag: Tensor, D: Tensor, h0: Optional[Tensor], ckpt: Tensor,
                    gy: Tensor, gh_last: Optional[Tensor], eps: float = 1e-6
                    ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(d_delta, d_s fp32, dB, dC, dlambda_alpha, dlambda_imag, dD fp32, dh0 fp32 or
    empty) of ssm_forward_dl_train given dL/dy and dL/dh_last."""
    ops = sf._dl_operands(delta, s, B, C, lambda_alpha, lambda_imag, D, h0)
    grads = sf.ssm_fused_dl_backward((*ops, ckpt), gy, gh_last, eps)
    dh0 = grads[-1]
    return (*grads[:-1], dh0 if dh0 is not None else B.new_empty(0, dtype=torch.float32))


@ssm_backward_dl.register_fake
def _(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, ckpt, gy, gh_last, eps=1e-6):
    b, t, d, n, _ = B.shape
    f32 = dict(dtype=torch.float32)
    return (B.new_empty(b, t, d, **f32), B.new_empty(b, t, d, **f32), torch.empty_like(B),
            torch.empty_like(C), B.new_empty(d, n, **f32), B.new_empty(d, n, 3, **f32),
            B.new_empty(d, **f32),
            B.new_empty(b, d, n, 4, **f32) if h0 is not None else B.new_empty(0, **f32))


def _ssm_train_setup(ctx, inputs, output):
    delta, s, B, C, la, li, D, h0, eps = inputs
    ctx.save_for_backward(delta, s, B, C, la, li, D, h0, output[2])
    ctx.eps = eps


def _ssm_train_backward(ctx, gy, gh_last, _gckpt):
    delta, s, B, C, la, li, D, h0, ckpt = ctx.saved_tensors
    d_delta, d_s, dB, dC, dla, dli, dD, dh0 = ssm_backward_dl(
        delta, s, B, C, la, li, D, h0, ckpt, gy, gh_last, ctx.eps)
    return (d_delta.to(delta.dtype), d_s.to(s.dtype), dB, dC, dla.to(la.dtype),
            dli.to(li.dtype), dD.to(D.dtype),
            None if h0 is None else dh0.to(h0.dtype), None)


register_autograd(f"{NS}::ssm_forward_dl_train", _ssm_train_backward,
                  setup_context=_ssm_train_setup)


# --- front of the SSM: delta = softplus(dt_raw), s = sigmoid(g_raw) * x --------

@custom_op(f"{NS}::ssm_front", mutates_args=())
def ssm_front(dt_raw: Tensor, g_raw: Tensor, x: Tensor) -> Tuple[Tensor, Tensor]:
    return sf.ssm_front(dt_raw, g_raw, x)


def _front_dtype(dt_raw, g_raw, x):
    return torch.promote_types(torch.promote_types(dt_raw.dtype, g_raw.dtype), x.dtype)


@ssm_front.register_fake
def _(dt_raw, g_raw, x):
    ct = _front_dtype(dt_raw, g_raw, x)
    return (dt_raw.new_empty(dt_raw.shape, dtype=ct), dt_raw.new_empty(dt_raw.shape, dtype=ct))


@custom_op(f"{NS}::ssm_front_backward", mutates_args=())
def ssm_front_backward(dt_raw: Tensor, g_raw: Tensor, x: Tensor, d_delta: Tensor,
                       d_s: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    dt, g, xv = sf._front_operands(dt_raw, g_raw, x)
    return sf._front_backward(dt, g, xv, d_delta, d_s)


@ssm_front_backward.register_fake
def _(dt_raw, g_raw, x, d_delta, d_s):
    ct = _front_dtype(dt_raw, g_raw, x)
    return tuple(dt_raw.new_empty(dt_raw.shape, dtype=ct) for _ in range(3))


def _front_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _front_bwd(ctx, g_delta, g_s):
    dt_raw, g_raw, x = ctx.saved_tensors
    d_dt, d_g, d_x = ssm_front_backward(dt_raw, g_raw, x, g_delta, g_s)
    return d_dt.to(dt_raw.dtype), d_g.to(g_raw.dtype), d_x.to(x.dtype)


register_autograd(f"{NS}::ssm_front", _front_bwd, setup_context=_front_setup)


# --- front + training walk as one operator ------------------------------------
# Under torch.compile with autograd, the front and the SSM's training walk are
# one operator so that the SSM's fp32 d_delta and d_s reach the front's
# backward without passing through delta's dtype (fp16/bf16 under autocast),
# as the eager _SsmFrontFusedDL does.

@custom_op(f"{NS}::ssm_front_forward_dl_train", mutates_args=())
def ssm_front_forward_dl_train(dt_raw: Tensor, g_raw: Tensor, x: Tensor, B: Tensor, C: Tensor,
                               lambda_alpha: Tensor, lambda_imag: Tensor, D: Tensor,
                               h0: Optional[Tensor] = None,
                               eps: float = 1e-6) -> Tuple[Tensor, Tensor, Tensor]:
    """(y, h_last fp32, fp32 checkpoints) of the training walk from the
    projections' outputs: delta = softplus(dt_raw), s = sigmoid(g_raw) * x."""
    dt, g, xv = sf._front_operands(dt_raw, g_raw, x)
    delta, s = sf._front_forward(dt, g, xv)
    y, h_last, saved = sf.ssm_fused_dl_train_forward(delta, s, B, C, lambda_alpha,
                                                     lambda_imag, D, h0, eps)
    return y, h_last, saved[-1]


@ssm_front_forward_dl_train.register_fake
def _(dt_raw, g_raw, x, B, C, lambda_alpha, lambda_imag, D, h0=None, eps=1e-6):
    b, t, d, n, _ = B.shape
    return (B.new_empty(b, t, d, 4), B.new_empty(b, d, n, 4, dtype=torch.float32),
            B.new_empty(*_ckpt_shape(B), dtype=torch.float32))


def _front_train_setup(ctx, inputs, output):
    dt_raw, g_raw, x, B, C, la, li, D, h0, eps = inputs
    ctx.save_for_backward(dt_raw, g_raw, x, B, C, la, li, D, h0, output[2])
    ctx.eps = eps


def _front_train_backward(ctx, gy, gh_last, _gckpt):
    dt_raw, g_raw, x, B, C, la, li, D, h0, ckpt = ctx.saved_tensors
    delta, s = ssm_front(dt_raw, g_raw, x)
    d_delta, d_s, dB, dC, dla, dli, dD, dh0 = ssm_backward_dl(
        delta, s, B, C, la, li, D, h0, ckpt, gy, gh_last, ctx.eps)
    # d_delta and d_s stay fp32 into the front's backward.
    d_dt, d_g, d_x = ssm_front_backward(dt_raw, g_raw, x, d_delta, d_s)
    return (d_dt.to(dt_raw.dtype), d_g.to(g_raw.dtype), d_x.to(x.dtype), dB, dC,
            dla.to(la.dtype), dli.to(li.dtype), dD.to(D.dtype),
            None if h0 is None else dh0.to(h0.dtype), None)


register_autograd(f"{NS}::ssm_front_forward_dl_train", _front_train_backward,
                  setup_context=_front_train_setup)


# --- Quaternion LayerNorm (quaternion_norm.py:119-245) ------------------------

@custom_op(f"{NS}::quaternion_layer_norm", mutates_args=())
def quaternion_layer_norm(q: Tensor, gamma: Tensor, beta: Tensor,
                          eps: float = 1e-5) -> Tuple[Tensor, Tensor, Tensor]:
    """(out in q's dtype, per-row mean and 1/std fp32 [B, T])."""
    out, mean, rstd, _, _ = _qln_forward(q, gamma, beta, eps, True)
    return out, mean, rstd


@quaternion_layer_norm.register_fake
def _(q, gamma, beta, eps=1e-5):
    b, t = q.shape[:2]
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            q.new_empty(b, t, dtype=torch.float32), q.new_empty(b, t, dtype=torch.float32))


@custom_op(f"{NS}::quaternion_layer_norm_backward", mutates_args=())
def quaternion_layer_norm_backward(q: Tensor, gamma: Tensor, mean: Tensor, rstd: Tensor,
                                   dout: Tensor, eps: float = 1e-5
                                   ) -> Tuple[Tensor, Tensor, Tensor]:
    """(dq in q's dtype, dgamma [D] fp32, dbeta [D, 4] fp32)."""
    return _qln_backward(nat.aligned16(q.detach()), nat.param_f32(gamma), mean, rstd, dout, eps)


@quaternion_layer_norm_backward.register_fake
def _(q, gamma, mean, rstd, dout, eps=1e-5):
    d = q.shape[2]
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            q.new_empty(d, dtype=torch.float32), q.new_empty(d, 4, dtype=torch.float32))


def _qln_setup(ctx, inputs, output):
    q, gamma, beta, eps = inputs
    ctx.save_for_backward(q, gamma, output[1], output[2])
    ctx.eps = eps
    ctx.beta_dtype = beta.dtype


def _qln_bwd(ctx, dout, _gmean, _grstd):
    q, gamma, mean, rstd = ctx.saved_tensors
    dq, dgamma, dbeta = quaternion_layer_norm_backward(q, gamma, mean, rstd, dout, ctx.eps)
    return dq.to(q.dtype), dgamma.to(gamma.dtype), dbeta.to(ctx.beta_dtype), None


register_autograd(f"{NS}::quaternion_layer_norm", _qln_bwd, setup_context=_qln_setup)


# --- causal depthwise conv + SiLU (causal_conv1d.py, block.py:137-140) --------

@custom_op(f"{NS}::causal_conv1d_silu", mutates_args=())
def causal_conv1d_silu(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    with torch.no_grad():
        return _ConvSiLU.apply(x, weight, bias)


@causal_conv1d_silu.register_fake
def _(x, weight, bias=None):
    return x.new_empty(x.shape)


@custom_op(f"{NS}::causal_conv1d_silu_backward", mutates_args=())
def causal_conv1d_silu_backward(x: Tensor, weight: Tensor, bias: Optional[Tensor],
                                gout: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """(dx in x's dtype, dweight [C, K] fp32, dbias [C] fp32)."""
    xv, xs = _rows_view(x.detach())
    C = x.shape[-1]
    w = nat.param_f32(weight).reshape(C, -1)
    b = None if bias is None else nat.param_f32(bias)
    return _conv_silu_backward(xv, xs, w, b, gout)


@causal_conv1d_silu_backward.register_fake
def _(x, weight, bias, gout):
    C = x.shape[-1]
    K = weight.shape[-1]
    return (x.new_empty(x.shape), x.new_empty(C, K, dtype=torch.float32),
            x.new_empty(C, dtype=torch.float32))


def _conv_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _conv_bwd(ctx, gout):
    x, weight, bias = ctx.saved_tensors
    dx, dw, db = causal_conv1d_silu_backward(x, weight, bias, gout)
    return (dx, dw.reshape(weight.shape).to(weight.dtype),
            None if bias is None else db.to(bias.dtype))


register_autograd(f"{NS}::causal_conv1d_silu", _conv_bwd, setup_context=_conv_setup)


# --- output gate: x + sigmoid(z[..., :d]) * y_real ------------------------------

def _gate_dtype(x, z, y_real):
    return torch.promote_types(torch.promote_types(x.dtype, z.dtype), y_real.dtype)


@custom_op(f"{NS}::out_gate", mutates_args=())
def out_gate(x: Tensor, z: Tensor, y_real: Tensor) -> Tensor:
    from .block import out_gate as _out_gate
    with torch.no_grad():
        return _out_gate(x, z, y_real)


@out_gate.register_fake
def _(x, z, y_real):
    return x.new_empty(x.shape, dtype=_gate_dtype(x, z, y_real))


@custom_op(f"{NS}::out_gate_backward", mutates_args=())
def out_gate_backward(x: Tensor, z: Tensor, y_real: Tensor,
                      dout: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """(dx, dz [z's shape], dy_real) in the promoted dtype."""
    _, zc, zs, yc, rows, d = _gate_operands(x, z, y_real)
    dx, dz, dy = _out_gate_backward(zc, zs, yc, rows, d, tuple(z.shape), dout)
    # dx is dout itself when dout is already in the operands' dtype and
    # aligned; an op's outputs may not alias its inputs.
    if dx.untyped_storage().data_ptr() == dout.untyped_storage().data_ptr():
        dx = dx.clone()
    return dx, dz, dy


@out_gate_backward.register_fake
def _(x, z, y_real, dout):
    ct = _gate_dtype(x, z, y_real)
    return (x.new_empty(x.shape, dtype=ct), z.new_empty(z.shape, dtype=ct),
            y_real.new_empty(y_real.shape, dtype=ct))


def _gate_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _gate_bwd(ctx, dout):
    x, z, y_real = ctx.saved_tensors
    dx, dz, dy = out_gate_backward(x, z, y_real, dout)
    return dx.to(x.dtype), dz.to(z.dtype), dy.to(y_real.dtype)


register_autograd(f"{NS}::out_gate", _gate_bwd, setup_context=_gate_setup)


OPS = (
    "quaternion_multiply", "quaternion_conjugate", "quaternion_inverse", "quaternion_norm",
    "cayley_discretization", "cumprod_scan", "ssm_forward_q", "ssm_step_q", "ssm_forward_dl",
    "ssm_forward_dl_train", "ssm_backward_dl", "ssm_front", "ssm_front_backward",
    "quaternion_layer_norm", "quaternion_layer_norm_backward", "causal_conv1d_silu",
    "causal_conv1d_silu_backward", "out_gate", "out_gate_backward",
)
