"""QuaternionMamba2Block on MI355X.

Drop-in for mambaqc/models/quaternion_mamba2_block.py:37-237: same constructor
signature, the same parameters created in the same order (identical weights
under the same seed, identical state_dict keys), and the same forward:

    xz = in_proj(x); x_in, z = chunk(xz)                    torch GEMM
    x_act = silu(conv1d(x_in))                              HIP: mqc_causal_conv_silu_fwd
    dt_raw, g_raw = dt_proj(x_act), gate_proj(x_act)        torch GEMMs
    delta = softplus(dt_raw); s = sigmoid(g_raw) * x_act    HIP: mqc_ssm_front_fwd
    B, C = B_proj(x_act), C_proj(x_act) as [B,T,D,S,4]      torch GEMMs (hipBLASLt)
    y = SSM(Cayley(delta * Lambda), B, s, C, D)             HIP: mqc_ssm_fused_fwd
      (16-bit inference of whole sequences: both lines as one HIP: mqc_ssm_fused_bc_fwd,
       kernel that never stores B or C)
    y = QuaternionLayerNorm(y)                              HIP: mqc_qln_fwd
    y_real = out_proj(y)                                    torch GEMM
    out = x + sigmoid(z[..., :d_model]) * y_real            HIP: mqc_out_gate_fwd
      (bf16 inference: both lines as one kernel,             HIP: mqc_out_proj_gate_fwd)

z, q and the quaternion S are never materialised: the SSM kernel discretises
in registers and takes the real selected signal s. When autograd is recording,
the front (softplus, sigmoid gate) + SSM, the conv + SiLU, QLN and gate run
as torch.autograd.Functions with HIP backward kernels (the reference's GPU
path has no backward: its Triton launches sit outside autograd); the GEMMs
use torch's autograd.

The gate uses z[..., :d_model]. The reference multiplies sigmoid(z), which has
d_inner = expand_factor * d_model features, by y_real, which has d_model
(block.py:157-161); that broadcast fails for any expand_factor != 1. The
reference's own Lite block gates with z[..., :d_model]
(quaternion_mamba2_lite_block.py:163), which is the rule used here. It is
identical to the reference whenever expand_factor == 1.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _native as nat
from .kernels.quaternion_norm import QuaternionLayerNorm
from .kernels import ssm_fused as _sf
from .kernels.ssm_fused import (fused_bc_eligible, ssm_forward_front_dl, ssm_forward_fused_bc,
                                ssm_forward_fused_dl, ssm_front)
from .layers.causal_conv1d import CausalConv1d, causal_conv1d_silu, causal_conv1d_silu_step_
from .layers.quaternion_linear import (quaternion_to_real_projection, real_to_quaternion_projection,
                                      skinny_eligible, skinny_linear)


def _gate_operands(x, z, y_real):
    """Operands in the result dtype: torch's promotion of x, z and y_real, as in
    the reference's x + sigmoid(z) * y_real (an fp32 residual stream under fp16
    autocast stays fp32)."""
    d = x.shape[-1]
    dtype = torch.promote_types(torch.promote_types(x.dtype, z.dtype), y_real.dtype)
    x = nat.aligned16(x.detach().to(dtype))
    z = z.detach().to(dtype)
    if z.stride(-1) != 1 or (z.dim() > 1 and not _rows_uniform(z)):
        z = z[..., :d].contiguous()
    y_real = nat.aligned16(y_real.detach().to(dtype))
    rows = x.numel() // d if d else 0
    zs = z.stride(-2) if z.dim() > 1 else z.shape[-1]
    return x, z, zs, y_real, rows, d


class _OutGateFunction(torch.autograd.Function):
    """out = x + sigmoid(z[..., :d]) * y_real with a HIP backward."""

    @staticmethod
    def forward(ctx, x, z, y_real):
        xc, zc, zs, yc, rows, d = _gate_operands(x, z, y_real)
        out = torch.empty_like(xc)
        nat.call("mqc_out_gate_fwd", xc, xc.data_ptr(), zc.data_ptr(), zs, yc.data_ptr(),
                 out.data_ptr(), rows, d, nat.dtype_code(xc), nat.stream_of(xc))
        ctx.save_for_backward(zc, yc)
        ctx.meta = (zs, rows, d, tuple(z.shape), x.dtype, z.dtype, y_real.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        zc, yc = ctx.saved_tensors
        zs, rows, d, zshape, t_x, t_z, t_y = ctx.meta
        dout, dz, dy = _out_gate_backward(zc, zs, yc, rows, d, zshape, dout)
        return dout.to(t_x), dz.to(t_z), dy.to(t_y)


def _out_gate_backward(zc, zs, yc, rows, d, zshape, dout):
    """(dx, dz [zshape], dy_real) in the operands' dtype from the forward's
    operands (_gate_operands). zc may have been narrowed to the first d
    columns: dz beyond d is zero either way."""
    dout = nat.aligned16(dout.to(yc.dtype))
    dz = torch.empty(zshape, device=yc.device, dtype=yc.dtype)
    dy = torch.empty_like(yc)
    nat.call("mqc_out_gate_bwd", yc, dout.data_ptr(), zc.data_ptr(), zs, yc.data_ptr(),
             dz.data_ptr(), dy.data_ptr(), rows, d, zshape[-1], nat.dtype_code(yc),
             nat.stream_of(yc))
    return dout, dz, dy


def out_gate(x: torch.Tensor, z: torch.Tensor, y_real: torch.Tensor) -> torch.Tensor:
    """x + sigmoid(z[..., :d]) * y_real for x, y_real [..., d] and z [..., >= d].

    z may be a strided view whose last axis is contiguous (the gate half of
    in_proj's output); it is read in place. Differentiable when autograd is
    recording.
    """
    d = x.shape[-1]
    assert y_real.shape == x.shape, f"y_real {tuple(y_real.shape)} vs x {tuple(x.shape)}"
    assert z.shape[:-1] == x.shape[:-1] and z.shape[-1] >= d
    if nat.compiling():
        return torch.ops.mambaqc.out_gate(x, z, y_real)
    nat.require_device("out_gate", x, z, y_real)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, z, y_real)):
        return _OutGateFunction.apply(x, z, y_real)
    xc, zc, zs, yc, rows, d = _gate_operands(x, z, y_real)
    out = torch.empty_like(xc)
    nat.call("mqc_out_gate_fwd", xc, xc.data_ptr(), zc.data_ptr(), zs, yc.data_ptr(),
             out.data_ptr(), rows, d, nat.dtype_code(xc), nat.stream_of(xc))
    return out


def out_proj_gate_eligible(x: torch.Tensor, z: torch.Tensor, y: torch.Tensor,
                           weight: torch.Tensor, bias: torch.Tensor | None) -> bool:
    """Whether out_proj_gate takes these operands: bf16 on a ROCm device, x
    [..., d_model] with d_model a multiple of 8, y [..., n, 4] with 4 n a multiple
    of 64, weight [d_model, 4 n], z's gate half readable as rows 16-byte aligned."""
    if not (x.is_cuda and z.is_cuda and y.is_cuda and weight.is_cuda):
        return False
    tensors = (x, z, y, weight) + (() if bias is None else (bias,))
    if any(t.dtype != torch.bfloat16 for t in tensors):
        return False
    d = x.shape[-1]
    k = y.shape[-2] * 4 if y.dim() >= 2 else 0
    if d % 8 or k % 64 or k == 0 or tuple(weight.shape) != (d, k):
        return False
    if z.shape[:-1] != x.shape[:-1] or z.shape[-1] < d or z.stride(-1) != 1:
        return False
    zs = z.stride(-2) if z.dim() > 1 else z.shape[-1]
    return (z.dim() == 1 or _rows_uniform(z)) and zs % 8 == 0 and z.data_ptr() % 16 == 0


def out_proj_gate(x: torch.Tensor, z: torch.Tensor, y: torch.Tensor, weight: torch.Tensor,
                  bias: torch.Tensor | None = None) -> torch.Tensor:
    """The block's output step in one HIP launch (inference, bf16):
    x + sigmoid(z[..., :d_model]) * out_proj(y), out_proj the quaternion -> real
    projection of y [..., n, 4] by weight [d_model, 4 n] (+ bias), its result rounded
    to bf16 as the projection stores it and gated without leaving the chip
    (mambaqc/layers/quaternion_linear.py:163-172 and
    mambaqc/models/quaternion_mamba2_block.py:157-164). z may be the strided gate
    half of in_proj's output; it is read in place."""
    nat.require_device("out_proj_gate", x, z, y, weight)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (x, z, y, weight, bias)):
        raise RuntimeError("out_proj_gate: inference only; run under torch.no_grad")
    if not out_proj_gate_eligible(x, z, y, weight, bias):
        raise ValueError("out_proj_gate: needs bf16 operands, d_model a multiple of 8, 4 n a "
                         "multiple of 64 and z rows 16-byte aligned")
    d = x.shape[-1]
    xc = nat.aligned16(x.detach())
    yc = nat.aligned16(y.detach())
    wc = nat.aligned16(weight.detach())
    bc = None if bias is None else bias.detach().contiguous()
    rows = xc.numel() // d
    zs = z.stride(-2) if z.dim() > 1 else z.shape[-1]
    out = torch.empty_like(xc)
    nat.call("mqc_out_proj_gate_fwd", xc, yc.data_ptr(), wc.data_ptr(), nat.ptr(bc),
             xc.data_ptr(), z.data_ptr(), zs, out.data_ptr(), rows, d, weight.shape[1],
             nat.BF16, nat.stream_of(xc))
    return out


def _rows_uniform(z: torch.Tensor) -> bool:
    """True when all leading axes of z collapse to a single row stride."""
    expected = z.stride(-2)
    for i in range(z.dim() - 2, 0, -1):
        expected *= z.shape[i]
        if z.shape[i - 1] > 1 and z.stride(i - 1) != expected:
            return False
    return True


# Inference only. The B and C projections ([batch, seq_len, d_inner, d_state, 4]
# each, 12.9 GB together in bf16 at batch 4, seq_len 2048, d_inner 1536,
# d_state 64) are materialised whole while both fit BC_WHOLE_MAX_BYTES. Past
# that the forward computes them d-slice by d-slice into two reused buffers of
# at most BC_SLICE_BYTES together and runs each slice's SSM from them, so the
# block's memory no longer grows with batch * seq_len * d_inner * d_state (at
# batch 1 and 262 144 tokens of the config-3 width, whole B and C would be
# 412 GB, more than one GPU's HBM). Whole is faster where it fits: at config 3
# the sliced form measured 18.5-18.9 ms against 16.7 ms for the GEMMs and SSM.
BC_WHOLE_MAX_BYTES = 32 << 30
BC_SLICE_BYTES = 2 << 30

# Inference in bf16 or fp16 from this many tokens per sequence on: the B/C projections and the
# SSM run as one kernel (mqc_ssm_fused_bc_fwd), B and C computed in 256-token tiles on
# chip and never stored. Shorter sequences (a decode step, short prompts) would fill one
# tile with a few tokens and keep the separate GEMMs. A batch of one runs the kernel with
# each half of the states in a workgroup of its own (ssm_forward_fused_bc's split), since
# one workgroup per d would re-stream more weight rows than the Infinity Cache holds.
# Block forward at the config-3 width, fused against unfused (one box): B1 T2048 4.63 /
# 4.91 ms, B1 T4096 9.00 / 9.47, B1 T16384 36.5 / 35.8, B1 T65536 145.3 / 144.5 (sliced);
# B2 T2048 8.81 / 9.16, B4 T2048 16.98 / 17.33 (one workgroup per d: B1 T2048 5.45 ms).
FUSED_BC_MIN_SEQ = 256
# The output step (out_proj + gate + residual) as one kernel (mqc_out_proj_gate_fwd) is
# opt-in (fuse_out=True). Back to back on operands resident in the chip's caches it beats
# out_proj (hipBLASLt) + the gate kernel at the config-3 shape (76.5 against 79.3 us), but
# inside the block its operands come from HBM: y just written, W, x and z evicted by the
# SSM's traffic, and there its two 28 KB stages per workgroup leave the K loop waiting on
# HBM latency (115-122 against 97-105 us with the caches flushed before each call;
# 109 against 92 us in a trace of the block).


def bc_slice_width(batch: int, seq_len: int, d_inner: int, d_state: int, elsize: int,
                   budget: int | None = None) -> int:
    """d's per slice so that one slice's B and C take at most `budget` bytes
    (None: BC_SLICE_BYTES), at least 1 and at most d_inner."""
    if budget is None:
        budget = BC_SLICE_BYTES
    per_d = 2 * batch * seq_len * d_state * 4 * elsize
    return max(1, min(d_inner, budget // max(per_d, 1)))


def _linear(layer: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """layer(x), on the library's skinny GEMM for decode-sized inputs."""
    if skinny_eligible(x, layer.weight, layer.bias):
        return skinny_linear(x, layer.weight, layer.bias)
    return layer(x)


def _linear_pair(a: nn.Linear, b: nn.Linear, x: torch.Tensor):
    """(a(x), b(x)), in one skinny launch for decode-sized inputs."""
    if skinny_eligible(x, a.weight, a.bias, b.weight, b.bias):
        return skinny_linear(x, a.weight, a.bias, b.weight, b.bias)
    return a(x), b(x)


def _bc_pair(bp, cp, x: torch.Tensor, d_state: int):
    """B_proj(x), C_proj(x) as [b, t, d, d_state, 4] (real -> quaternion maps),
    in one skinny launch for decode-sized inputs with weights small enough."""
    b, t, D = x.shape
    bb = None if bp.bias is None else bp.bias.reshape(-1)
    cb = None if cp.bias is None else cp.bias.reshape(-1)
    if skinny_eligible(x, bp.weight, bb, cp.weight, cb):
        Bq, Cq = skinny_linear(x, bp.weight, bb, cp.weight, cb)
    else:
        Bq, Cq = bp(x), cp(x)
    return Bq.view(b, t, D, d_state, 4), Cq.view(b, t, D, d_state, 4)


def _out_proj(op, y: torch.Tensor) -> torch.Tensor:
    """out_proj(y) (quaternion -> real), on the skinny GEMM for decode-sized inputs."""
    y2 = y.reshape(*y.shape[:-2], y.shape[-2] * 4)
    if skinny_eligible(y2, op.weight, op.bias):
        return skinny_linear(y2, op.weight, op.bias)
    return op(y)


class _SlicedBCTrain(torch.autograd.Function):
    """The front and the SSM of the block with the B and C projections computed
    d-slice by d-slice, differentiable, without B, C, dB or dC ever whole.

    Forward: delta, s from the front (HIP); per slice, the two projection GEMMs
    into reused buffers and the SSM's inference walk over that slice. Only the
    inputs are saved. Backward, per slice: the two GEMMs again, the SSM's
    training walk (its fp32 checkpoints, slice-sized), the SSM backward, then
    the slice's weight gradients (dB_s^T x, written in place) and its share of
    dx (dB_s W_s, accumulated in fp32); finally the front's backward. Against
    whole projections this costs two GEMMs and one SSM walk more per step and
    holds O(slice) memory for everything of size batch x seq_len x d_inner x
    d_state.
    """

    @staticmethod
    def forward(ctx, x_act, dt_raw, g_raw, wb, wc, lam_a, lam_i, dskip, h0, width, d_state,
                eps, dtype):
        b, t, D = x_act.shape
        S = d_state
        dt, g, xv = _sf._front_operands(dt_raw, g_raw, x_act)
        delta, s = _sf._front_forward(dt, g, xv)
        x2 = x_act.detach().reshape(b * t, D).to(dtype)
        la, li, dv = (nat.param_f32(p) for p in (lam_a, lam_i, dskip))
        buf = torch.empty(2, b * t * width * S * 4, device=x_act.device, dtype=dtype)
        y = torch.empty(b, t, D, 4, device=x_act.device, dtype=dtype)
        h_last = torch.empty(b, D, S, 4, device=x_act.device, dtype=torch.float32)
        with torch.autocast(x_act.device.type, enabled=False):
            _SlicedBCTrain._walks(x2, wb, wc, buf, delta, s, la, li, dv, h0, y, h_last, width,
                                  S, eps, dtype)
        ctx.save_for_backward(x_act, dt_raw, g_raw, wb, wc, lam_a, lam_i, dskip, h0)
        ctx.meta = (width, S, eps, dtype)
        return y, h_last

    @staticmethod
    def _walks(x2, wb, wc, buf, delta, s, la, li, dv, h0, y, h_last, width, S, eps, dtype):
        b, t, D = delta.shape
        for d0 in range(0, D, width):
            n = min(width, D - d0)
            bs, cs = _SlicedBCTrain._bc(x2, wb, wc, buf, d0, n, S, dtype)
            ys, hs = ssm_forward_fused_dl(
                delta[:, :, d0:d0 + n], s[:, :, d0:d0 + n], bs.view(b, t, n, S, 4),
                cs.view(b, t, n, S, 4), la[d0:d0 + n], li[d0:d0 + n], dv[d0:d0 + n], eps=eps,
                h0=None if h0 is None else h0[:, d0:d0 + n].detach(), return_state=True)
            y[:, :, d0:d0 + n] = ys
            h_last[:, d0:d0 + n] = hs

    @staticmethod
    def _bc(x2, wb, wc, buf, d0, n, S, dtype):
        r0, r1 = d0 * S * 4, (d0 + n) * S * 4
        m = x2.shape[0]
        bs = buf[0, : m * n * S * 4].view(m, n * S * 4)
        cs = buf[1, : m * n * S * 4].view(m, n * S * 4)
        torch.mm(x2, wb.detach()[r0:r1].to(dtype).t(), out=bs)
        torch.mm(x2, wc.detach()[r0:r1].to(dtype).t(), out=cs)
        return bs, cs

    @staticmethod
    def backward(ctx, gy, gh_last):
        x_act, dt_raw, g_raw, wb, wc, lam_a, lam_i, dskip, h0 = ctx.saved_tensors
        width, S, eps, dtype = ctx.meta
        b, t, D = x_act.shape
        m = b * t
        dev = x_act.device
        dt, g, xv = _sf._front_operands(dt_raw, g_raw, x_act)
        delta, s = _sf._front_forward(dt, g, xv)
        x2 = x_act.detach().reshape(m, D).to(dtype)
        la, li, dv = (nat.param_f32(p) for p in (lam_a, lam_i, dskip))
        f32 = torch.float32
        wide = {} if dtype == f32 else {"out_dtype": f32}
        d_delta = torch.empty(b, t, D, device=dev, dtype=f32)
        d_s = torch.empty(b, t, D, device=dev, dtype=f32)
        dla = torch.empty(D, S, device=dev, dtype=f32)
        dli = torch.empty(D, S, 3, device=dev, dtype=f32)
        dD = torch.empty(D, device=dev, dtype=f32)
        dh0 = None if h0 is None else torch.empty(b, D, S, 4, device=dev, dtype=f32)
        # Weight gradients and the projections' share of dx only where asked
        # for (frozen projections skip two GEMMs per slice each).
        need_x, need_wb, need_wc = (ctx.needs_input_grad[i] for i in (0, 3, 4))
        dwb = torch.empty(wb.shape, device=dev, dtype=f32) if need_wb else None
        dwc = torch.empty(wc.shape, device=dev, dtype=f32) if need_wc else None
        dx2 = torch.zeros(m, D, device=dev, dtype=f32) if need_x else None
        buf = torch.empty(2, m * width * S * 4, device=dev, dtype=dtype)
        gy = gy if gy is not None else torch.zeros(b, t, D, 4, device=dev, dtype=dtype)
        for d0 in range(0, D, width):
            n = min(width, D - d0)
            r0, r1 = d0 * S * 4, (d0 + n) * S * 4
            bs, cs = _SlicedBCTrain._bc(x2, wb, wc, buf, d0, n, S, dtype)
            _, _, saved = _sf.ssm_fused_dl_train_forward(
                delta[:, :, d0:d0 + n], s[:, :, d0:d0 + n], bs.view(b, t, n, S, 4),
                cs.view(b, t, n, S, 4), la[d0:d0 + n], li[d0:d0 + n], dv[d0:d0 + n],
                None if h0 is None else h0[:, d0:d0 + n].detach(), eps)
            dd, dss, dB, dC, dla_s, dli_s, dD_s, dh0_s = _sf.ssm_fused_dl_backward(
                saved, gy[:, :, d0:d0 + n],
                None if gh_last is None else gh_last[:, d0:d0 + n], eps)
            del saved
            d_delta[:, :, d0:d0 + n] = dd
            d_s[:, :, d0:d0 + n] = dss
            dla[d0:d0 + n] = dla_s
            dli[d0:d0 + n] = dli_s
            dD[d0:d0 + n] = dD_s
            if dh0 is not None:
                dh0[:, d0:d0 + n] = dh0_s
            dB2 = dB.view(m, n * S * 4)
            dC2 = dC.view(m, n * S * 4)
            if need_wb:
                torch.mm(dB2.t(), x2, **wide, out=dwb[r0:r1])
            if need_wc:
                torch.mm(dC2.t(), x2, **wide, out=dwc[r0:r1])
            if need_x:
                dx2.add_(torch.mm(dB2, wb.detach()[r0:r1].to(dtype), **wide))
                dx2.add_(torch.mm(dC2, wc.detach()[r0:r1].to(dtype), **wide))
            del dB, dC, dB2, dC2
        d_dt, d_g, d_x = _sf._front_backward(dt, g, xv, d_delta, d_s)
        dx = d_x.float().add_(dx2.view(b, t, D)).to(x_act.dtype) if need_x else None
        return (dx, d_dt.to(dt_raw.dtype), d_g.to(g_raw.dtype),
                None if dwb is None else dwb.to(wb.dtype),
                None if dwc is None else dwc.to(wc.dtype), dla.to(lam_a.dtype), dli.to(lam_i.dtype),
                dD.to(dskip.dtype), None if dh0 is None else dh0.to(h0.dtype),
                None, None, None, None)


class QuaternionMamba2Block(nn.Module):
    """One Quaternion Mamba-2 block. Input and output: [batch, seq_len, d_model].

    bc_slice_d (attribute, not a parameter): None lets the forward slice the
    B/C projections only when whole ones would exceed BC_WHOLE_MAX_BYTES; an
    int forces slices of that many d's; 0 never slices. Inference slices run
    the SSM per slice; training slices (_SlicedBCTrain) also recompute each
    slice's projections in the backward.

    fuse_bc (attribute): None runs inference (no autograd) with the B/C
    projections fused into the SSM kernel (ssm_forward_fused_bc) where that
    kernel applies (bf16 or fp16 operands, or autocast to either; bias-free
    projections, d_inner a multiple of 64, even d_state <= 64) and sequences have at least FUSED_BC_MIN_SEQ tokens; True
    also for shorter ones; False never. A forced bc_slice_d takes precedence.

    fuse_out (attribute): True runs the output step of bf16 inference (out_proj,
    gate, residual) as one kernel (out_proj_gate) where it applies; None (the
    default) and False run out_proj, then out_gate.
    """

    def __init__(self, d_model: int, d_state: int = 64, d_conv: int = 4,
                 expand_factor: int = 2, dt_rank: str | int = "auto", bias: bool = False):
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.d_conv = d_conv
        self.d_inner = d_model * expand_factor
        self.dt_rank = max(16, d_model // 16) if dt_rank == "auto" else dt_rank
        D = self.d_inner

        # Parameter creation order fixes the RNG stream (block.py:78-122).
        self.in_proj = nn.Linear(d_model, 2 * D, bias=bias)
        self.conv1d = CausalConv1d(D, kernel_size=d_conv, bias=True)
        self.Lambda_alpha = nn.Parameter(torch.randn(D, d_state) * 0.5 + 1.0)
        self.Lambda_imag = nn.Parameter(torch.randn(D, d_state, 3) * 0.1)
        self.dt_proj = nn.Linear(D, D, bias=True)
        self.B_proj = real_to_quaternion_projection(D, D * d_state, bias=False)
        self.C_proj = real_to_quaternion_projection(D, D * d_state, bias=False)
        self.D = nn.Parameter(torch.ones(D))
        self.gate_proj = nn.Linear(D, D, bias=False)
        self.norm = QuaternionLayerNorm(D, eps=1e-5)
        self.out_proj = quaternion_to_real_projection(D, d_model, bias=bias)
        self.bc_slice_d: int | None = None
        self.fuse_bc: bool | None = None
        self.fuse_out: bool | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xz = _linear(self.in_proj, x)
        x_in, z = xz.chunk(2, dim=-1)
        conv = self.conv1d.conv
        x_act = causal_conv1d_silu(x_in, conv.weight, conv.bias)
        y = self._ssm_forward(x_act)
        y = self.norm(y)
        return self._output_step(x, z, y)

    def _output_step(self, x: torch.Tensor, z: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """x + sigmoid(z[..., :d_model]) * out_proj(y): one fused launch for bf16
        inference where it applies (fuse_out), else out_proj then out_gate."""
        op = self.out_proj
        if (self.fuse_out and not nat.compiling()
                and not (torch.is_grad_enabled() and (y.requires_grad or x.requires_grad
                                                      or op.weight.requires_grad))
                and out_proj_gate_eligible(x, z, y, op.weight, op.bias)):
            return out_proj_gate(x, z, y, op.weight, op.bias)
        return out_gate(x, z, _out_proj(op, y))

    def forward_with_state(self, x: torch.Tensor, state=None):
        """forward() continued from a recurrent state; returns (out, new_state).

        state = (conv_tail, h): conv_tail [batch, d_conv - 1, d_inner] holds the
        last d_conv - 1 conv inputs, h [batch, d_inner, d_state, 4] the SSM
        state, in fp32 whatever the model dtype (the precision the walk
        carries it in). None starts from zeros, where the result equals forward(x).
        Feeding a sequence in pieces gives the same outputs as feeding it whole
        (up to rounding), which is what recurrent decoding relies on.
        """
        xz = _linear(self.in_proj, x)
        x_in, z = xz.chunk(2, dim=-1)
        b, _, D = x_in.shape
        k = self.d_conv - 1
        if state is None:
            tail, h0 = x_in.new_zeros(b, k, D), None
        else:
            tail, h0 = state
        xc = torch.cat([tail.to(x_in.dtype), x_in], dim=1)
        conv = self.conv1d.conv
        # The tail rows stand in for the zero padding: outputs from row k on
        # are the continued convolution.
        x_act = causal_conv1d_silu(xc, conv.weight, conv.bias)[:, k:].contiguous()
        y, h = self._ssm_forward(x_act, h0=h0, return_state=True)
        y_real = _out_proj(self.out_proj, self.norm(y))
        return out_gate(x, z, y_real), (xc[:, xc.shape[1] - k:], h)

    def step_state_(self, x: torch.Tensor, state) -> torch.Tensor:
        """One token per sequence, x [batch, 1, d_model], continued from state =
        (conv_tail, h), which is updated in place to the state after x; returns
        out [batch, 1, d_model], equal to forward_with_state(x, state)[0]. The
        recurrent decode step, without autograd: conv_tail contiguous
        [batch, d_conv - 1, d_inner] in x's dtype, h contiguous fp32
        [batch, d_inner, d_state, 4]. The conv continues from the tail in one
        kernel that also shifts it, and the SSM writes its final state over h, so
        the step copies no state."""
        tail, h = state
        xz = _linear(self.in_proj, x)
        x_in, z = xz.chunk(2, dim=-1)
        conv = self.conv1d.conv
        x_act = causal_conv1d_silu_step_(x_in, tail, conv.weight, conv.bias)
        dt_raw, g_raw = _linear_pair(self.dt_proj, self.gate_proj, x_act)
        Bq, Cq = _bc_pair(self.B_proj, self.C_proj, x_act, self.d_state)
        y = _sf.ssm_forward_front_dl_state_(dt_raw, g_raw, x_act, Bq, Cq, self.Lambda_alpha,
                                            self.Lambda_imag, self.D, h, eps=1e-6)
        y_real = _out_proj(self.out_proj, self.norm(y))
        return out_gate(x, z, y_real)

    def _ssm_forward(self, x: torch.Tensor, h0: torch.Tensor | None = None,
                     return_state: bool = False):
        """x: [batch, seq_len, d_inner] (real) -> y: [batch, seq_len, d_inner, 4]."""
        b, t, D = x.shape
        recording = torch.is_grad_enabled() and (
            x.requires_grad or (h0 is not None and h0.requires_grad)
            or any(p.requires_grad for p in self.parameters()))
        width = self._bc_slice_width(x, recording)
        dt_raw, g_raw = _linear_pair(self.dt_proj, self.gate_proj, x)
        if not recording and self._use_fused_bc(x):
            delta, s = ssm_front(dt_raw, g_raw, x)
            # Under autocast the projections' operands in its dtype, as F.linear casts them.
            dt = self._gemm_dtype(x)
            xf, wb, wc = (t if t.dtype == dt else t.to(dt)
                          for t in (x, self.B_proj.weight, self.C_proj.weight))
            return ssm_forward_fused_bc(xf, wb, wc, delta, s, self.Lambda_alpha, self.Lambda_imag,
                                        self.D, eps=1e-6, h0=h0, return_state=return_state)
        if width:
            if recording:
                if self.B_proj.bias is not None or self.C_proj.bias is not None:
                    raise ValueError("sliced B/C projections take bias-free B_proj and C_proj")
                nat.require_device("QuaternionMamba2Block", x, dt_raw, g_raw)
                y, h = _SlicedBCTrain.apply(
                    x, dt_raw, g_raw, self.B_proj.weight, self.C_proj.weight, self.Lambda_alpha,
                    self.Lambda_imag, self.D, h0, width, self.d_state, 1e-6, self._gemm_dtype(x))
                return (y, h) if return_state else y
            return self._ssm_forward_sliced(x, dt_raw, g_raw, width, h0, return_state)
        Bq, Cq = _bc_pair(self.B_proj, self.C_proj, x, self.d_state)
        return ssm_forward_front_dl(dt_raw, g_raw, x, Bq, Cq, self.Lambda_alpha,
                                    self.Lambda_imag, self.D, eps=1e-6, h0=h0,
                                    return_state=return_state)

    def _use_fused_bc(self, x: torch.Tensor) -> bool:
        """Whether this inference forward runs the B/C projections fused into the
        SSM kernel (fuse_bc; the class docstring)."""
        if self.fuse_bc is False or (self.bc_slice_d or 0) > 0:
            return False
        if self.B_proj.bias is not None or self.C_proj.bias is not None:
            return False
        if self.fuse_bc is None and x.shape[1] < FUSED_BC_MIN_SEQ:
            return False
        dt = (torch.get_autocast_dtype(x.device.type)
              if torch.is_autocast_enabled(x.device.type) else None)
        return fused_bc_eligible(x, self.B_proj.weight, self.C_proj.weight, self.d_state, dt)

    def _gemm_dtype(self, x: torch.Tensor) -> torch.dtype:
        if torch.is_autocast_enabled(x.device.type):
            return torch.get_autocast_dtype(x.device.type)
        return x.dtype

    def _bc_slice_width(self, x: torch.Tensor, recording: bool | None = None) -> int:
        """d's per B/C slice for this input, 0 for whole projections.
        recording: whether autograd records this forward (None: judged from x
        and the parameters)."""
        forced = self.bc_slice_d
        if forced == 0:
            return 0
        if recording is None:
            recording = torch.is_grad_enabled() and (x.requires_grad or any(
                p.requires_grad for p in self.parameters()))
        if forced is not None:
            if forced < 0:
                raise ValueError(f"bc_slice_d must be >= 0 or None, got {forced}")
            if recording:
                _sf._require_trainable_state(torch.empty(0, self.d_state, 4))
            return min(int(forced), self.d_inner)
        if self.B_proj.bias is not None or self.C_proj.bias is not None:
            return 0
        if recording and self.d_state > _sf.SSM_BWD_MAX_STATE:
            return 0
        b, t, D = x.shape
        el = 4 if self._gemm_dtype(x) == torch.float32 else 2
        if 2 * b * t * D * self.d_state * 4 * el <= BC_WHOLE_MAX_BYTES:
            return 0
        return bc_slice_width(b, t, D, self.d_state, el)

    def _ssm_forward_sliced(self, x, dt_raw, g_raw, width, h0, return_state):
        """The SSM with B and C computed `width` d's at a time into two reused
        buffers: per slice, the two projection GEMMs (rows of the weights as
        stored) and the SSM over that slice's d's, from that slice's h0.
        Each (b, d) state depends only on its own d's B, C, delta and s, so
        the slices are independent."""
        if self.B_proj.bias is not None or self.C_proj.bias is not None:
            raise ValueError("sliced B/C projections take bias-free B_proj and C_proj")
        b, t, D = x.shape
        S = self.d_state
        delta, s = ssm_front(dt_raw, g_raw, x)
        dtype = self._gemm_dtype(x)
        x2 = x.reshape(b * t, D).to(dtype)
        wb, wc = self.B_proj.weight.detach(), self.C_proj.weight.detach()
        # fp32 forms of the SSM parameters, converted once (cached) and sliced.
        la, li, dv = (nat.param_f32(p) for p in (self.Lambda_alpha, self.Lambda_imag, self.D))
        per = b * t * width * S * 4
        buf = torch.empty(2, per, device=x.device, dtype=dtype)
        y = torch.empty(b, t, D, 4, device=x.device, dtype=dtype)
        h_last = (torch.empty(b, D, S, 4, device=x.device, dtype=torch.float32)
                  if return_state else None)
        with torch.autocast(x.device.type, enabled=False):
            for d0 in range(0, D, width):
                n = min(width, D - d0)
                r0, r1 = d0 * S * 4, (d0 + n) * S * 4
                bs = buf[0, : b * t * n * S * 4].view(b * t, n * S * 4)
                cs = buf[1, : b * t * n * S * 4].view(b * t, n * S * 4)
                torch.mm(x2, wb[r0:r1].to(dtype).t(), out=bs)
                torch.mm(x2, wc[r0:r1].to(dtype).t(), out=cs)
                out = ssm_forward_fused_dl(
                    delta[:, :, d0:d0 + n], s[:, :, d0:d0 + n], bs.view(b, t, n, S, 4),
                    cs.view(b, t, n, S, 4), la[d0:d0 + n], li[d0:d0 + n], dv[d0:d0 + n],
                    eps=1e-6,
                    h0=None if h0 is None else h0[:, d0:d0 + n], return_state=return_state)
                if return_state:
                    out, h_slice = out
                    h_last[:, d0:d0 + n] = h_slice
                y[:, :, d0:d0 + n] = out
        return (y, h_last) if return_state else y

    def extra_repr(self) -> str:
        return (f"d_model={self.d_model}, d_state={self.d_state}, d_inner={self.d_inner}, "
                f"d_conv={self.d_conv}, dt_rank={self.dt_rank}")
