"""Linear maps between real and quaternion feature spaces.

Same parameters, initialisation and forward semantics as
mambaqc/layers/quaternion_linear.py:16-266, so state dicts and seeded weights
are interchangeable with the reference. The maps are dense GEMMs and run as
torch F.linear (hipBLASLt on MI355X); the quaternion layout is a view:
    real -> quaternion: [..., in] @ W^T -> [..., out/4, 4]   (+ bias [out/4, 4])
    quaternion -> real: [..., n, 4] -> [..., 4n] @ W^T       (+ bias [out])
    quaternion -> quaternion: the real block map of the flattened components.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _native as nat

_KINDS = ("real", "quaternion")

# Bound on the weight bytes one GEMM launch streams in wide_linear. MI355X's
# Infinity Cache (the memory-side cache in front of HBM) holds 256 MB: a weight
# block of this size stays resident while every token tile of the launch reads
# it, where a single launch over a 1.2 GB weight (the config-3 B/C projections)
# re-streams the weight from HBM for every row of token tiles. Measured at
# M 8192, N 393216, K 1536 (6 blocks of 192 MiB): forward 7.57 -> 7.28 ms in
# bf16 and 7.72 -> 7.48 ms in fp16, bit-identical outputs; weight gradient
# 9.20 -> 8.87 ms; input gradient (K blocks) 8.77 -> ~8.5 ms.
WIDE_LINEAR_CHUNK_BYTES = 192 << 20
# Below this many token rows a single launch reads the weight about once (one
# row of output tiles), and extra launches only add launch overhead (the
# recurrent decode step has 4 rows).
WIDE_LINEAR_MIN_ROWS = 1024


def _blocks(n: int, k: int, elsize: int):
    """[n0, n1) blocks of the n weight rows (k elements each), every block at
    most WIDE_LINEAR_CHUNK_BYTES and starting on a 256-row boundary."""
    chunks = -(-(n * k * elsize) // WIDE_LINEAR_CHUNK_BYTES)
    step = -(-n // chunks)
    step = -(-step // 256) * 256
    return [(n0, min(n, n0 + step)) for n0 in range(0, n, step)]


# The input gradient dx = gy W is a sum over the weight's rows. Launched one
# row block at a time, each GEMM has only ⌈M/tile⌉ × ⌈K/tile⌉ output tiles
# (about one per CU at the config-4 shape), so every launch ends with a
# partial wave of tiles. One batched GEMM over equal row blocks (fp32 partial
# products, summed afterwards) runs them all in one launch. Measured at
# M 8192, N 393216, K 1536 on MI355X: 8 blocks in one launch 7.94-7.99 ms
# (fp16) and 7.68-7.72 ms (bf16), against 8.55-8.64 and 8.17-8.29 ms for six
# launches of 192 MiB blocks; 12 and 16 blocks 7.97-8.08 ms (fp16), 6 blocks
# in one launch 9.54 ms.
WIDE_DX_MIN_BATCHES = 8


def _dx_batches(n: int, k: int, elsize: int) -> int:
    """Number of equal row blocks for the batched input gradient: the first
    count from max(WIDE_DX_MIN_BATCHES, the forward's block count) up to four
    times that which divides n, or 0 when none does (the blocked loop runs)."""
    nb0 = max(WIDE_DX_MIN_BATCHES, len(_blocks(n, k, elsize)))
    for nb in range(nb0, 4 * nb0 + 1):
        if n % nb == 0:
            return nb
    return 0


def _wide_forward(x2: torch.Tensor, weight: torch.Tensor, out2: torch.Tensor) -> None:
    for n0, n1 in _blocks(*weight.shape, weight.element_size()):
        torch.mm(x2, weight[n0:n1].t(), out=out2[:, n0:n1])


class _WideLinearFunction(torch.autograd.Function):
    """y = x W^T by column blocks; the backward splits the same way:
    dW by row blocks (each dW[n0:n1] = gy[:, n0:n1]^T x, written in place) and
    dx as a sum over K blocks with fp32 partials, rounded once (the partials
    from one batched GEMM over equal blocks where WIDE_DX_MIN_BATCHES or more
    of them divide the weight's rows, else one GEMM per block).

    `dtype` is the GEMMs' operand dtype (autocast's), or None to use the
    inputs' own. The casts happen inside the node, so an fp32 weight under
    16-bit autocast gets its gradient straight from the GEMMs in fp32 (16-bit
    operands, fp32 accumulation and output) instead of a 16-bit gradient and a
    separate cast pass over it.
    """

    @staticmethod
    def forward(ctx, x, weight, dtype):
        n, k = weight.shape
        xd = x if dtype is None else x.to(dtype)
        wd = weight if dtype is None else weight.to(dtype)
        x2 = xd.reshape(-1, k)
        out = torch.empty(*x.shape[:-1], n, device=x.device, dtype=wd.dtype)
        _wide_forward(x2, wd, out.view(-1, n))
        ctx.save_for_backward(x2, wd)
        ctx.x_shape = x.shape
        ctx.dtypes = (x.dtype, weight.dtype)
        return out

    @staticmethod
    def backward(ctx, gy):
        x2, wd = ctx.saved_tensors
        x_dtype, w_dtype = ctx.dtypes
        n, k = wd.shape
        gy2 = gy.to(wd.dtype).reshape(-1, n)
        blocks = _blocks(n, k, wd.element_size())
        wide = {} if wd.dtype == torch.float32 else {"out_dtype": torch.float32}
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dense = gy2.is_contiguous() and wd.is_contiguous()
            nb = _dx_batches(n, k, wd.element_size()) if dense else 0
            if nb:
                # [nb, rows, n/nb] x [nb, n/nb, k] -> nb fp32 partials of dx.
                rows, step = gy2.shape[0], n // nb
                parts = torch.bmm(gy2.view(rows, nb, step).transpose(0, 1),
                                  wd.view(nb, step, k), **wide)
                acc = parts.sum(0)
            else:
                acc = None
                for n0, n1 in blocks:
                    part = torch.mm(gy2[:, n0:n1], wd[n0:n1], **wide)
                    acc = part if acc is None else acc.add_(part)
            dx = acc.to(x_dtype).view(ctx.x_shape)
        if ctx.needs_input_grad[1]:
            # fp32 straight from the GEMMs for an fp32 weight; otherwise in the
            # operand dtype.
            fp32_out = w_dtype == torch.float32
            dw = torch.empty(n, k, device=wd.device, dtype=torch.float32 if fp32_out else wd.dtype)
            for n0, n1 in blocks:
                torch.mm(gy2[:, n0:n1].t(), x2, **(wide if fp32_out else {}), out=dw[n0:n1])
            dw = dw.to(w_dtype)
        return dx, dw, None


def wide_linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.linear(x, weight) without bias, computed as column blocks of the
    output whose weight rows fit WIDE_LINEAR_CHUNK_BYTES, each written in place
    into one output tensor by its own GEMM (and differentiable, with the
    backward blocked the same way).

    Used on a GPU when the weight exceeds the bound and x has at least
    WIDE_LINEAR_MIN_ROWS rows; everything else takes F.linear. Under autocast
    the operands are cast to the autocast dtype, as F.linear's autocast rule
    does. Each output element is the same K-reduction as in one launch.
    """
    n, k = weight.shape
    rows = x.numel() // k if k else 0
    if (n * k * weight.element_size() <= WIDE_LINEAR_CHUNK_BYTES or rows < WIDE_LINEAR_MIN_ROWS
            or not x.is_cuda or not weight.is_cuda or torch.compiler.is_compiling()):
        # (Under torch.compile the product is left to the compiler as one GEMM.)
        return F.linear(x, weight)
    dtype = None
    if torch.is_autocast_enabled(x.device.type):
        dtype = torch.get_autocast_dtype(x.device.type)
    elif x.dtype != weight.dtype:
        return F.linear(x, weight)  # raises torch's dtype error
    with torch.autocast(x.device.type, enabled=False):
        if torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad):
            return _WideLinearFunction.apply(x, weight, dtype)
        if dtype is not None:
            x, weight = x.to(dtype), weight.to(dtype)
        x2 = x.reshape(-1, k)
        out = torch.empty(*x.shape[:-1], n, device=x.device, dtype=x.dtype)
        _wide_forward(x2, weight, out.view(-1, n))
        return out


# Decode-sized products (at most this many token rows, no autograd, 16-bit)
# run on the library's skinny GEMM (mqc_gemm_skinny_nt), which takes a pair of
# weights sharing the input in one launch. Measured at 4 rows on MI355X: a pair
# of [1024 x 1024] weights 6.3 us in one launch against about 6.6 us per weight
# through hipBLASLt, [131072 x 1024] pairs 95-98 against 99.7 us.
SKINNY_MAX_ROWS = 16
# With at most SKINNY_WIDE_MAX_ROWS token rows and K a multiple of 64, the
# library streams large weights in its wide mode (whole 128-byte lines per load,
# VALU dot products), faster than hipBLASLt's GEMV: the base preset's
# [393216 x 1536] B/C pair at 4 rows 386-392 us against 427 us (the base
# preset's decode step 5.73 -> 5.30 ms). Other shapes keep hipBLASLt for
# weights above SKINNY_MAX_WEIGHT_BYTES: in 16-row MFMA tiles that pair took
# 420 us against 409 us.
SKINNY_WIDE_MAX_ROWS = 8
SKINNY_MAX_WEIGHT_BYTES = 512 << 20


def _skinny_wide(rows: int, K: int) -> bool:
    """Whether mqc_gemm_skinny_nt may stream a large weight in its wide mode:
    at most SKINNY_WIDE_MAX_ROWS rows, K a multiple of 64, and X (rows padded
    to a power of two) within its 64 KiB of LDS."""
    padded = 1 << max(rows - 1, 0).bit_length()
    return rows <= SKINNY_WIDE_MAX_ROWS and K % 64 == 0 and padded * K * 2 <= (64 << 10)


def skinny_eligible(x: torch.Tensor, *params) -> bool:
    """Whether F.linear(x, w, b) for every (w, b) in params (flat: w1, b1, w2,
    b2, ...) may run on mqc_gemm_skinny_nt: few rows, 16-bit operands of one
    dtype, K a multiple of 32, dense weights (of at most SKINNY_MAX_WEIGHT_BYTES
    unless the wide mode applies), nothing recording autograd, no autocast, not
    under torch.compile."""
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16) or x.dim() < 1:
        return False
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if not (0 < rows <= SKINNY_MAX_ROWS) or K % 32 or rows * (K + 8) * 2 > (64 << 10):
        return False
    if torch.compiler.is_compiling() or torch.is_autocast_enabled(x.device.type):
        return False
    tensors = [x] + [p for p in params if p is not None]
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return False
    wide = _skinny_wide(rows, K)
    for w, b in zip(params[0::2], params[1::2]):
        if (w.dtype != x.dtype or w.device != x.device or w.dim() != 2 or w.shape[1] != K
                or not w.is_contiguous() or w.data_ptr() % 16
                or (w.numel() * 2 > SKINNY_MAX_WEIGHT_BYTES and not wide)):
            return False
        if b is not None and (b.dtype != x.dtype or b.numel() != w.shape[0]
                              or not b.is_contiguous()):
            return False
    return True


def skinny_linear(x: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor | None = None,
                  w2: torch.Tensor | None = None, b2: torch.Tensor | None = None):
    """F.linear(x, w1, b1) and, with w2, F.linear(x, w2, b2) in one launch of
    mqc_gemm_skinny_nt; for inputs skinny_eligible accepts. Returns y1 or
    (y1, y2), [..., N] in x's dtype (bias added in fp32 before the rounding)."""
    K = x.shape[-1]
    x2 = nat.aligned16(x.reshape(-1, K))
    M = x2.shape[0]
    lead = x.shape[:-1]
    y1 = torch.empty(*lead, w1.shape[0], device=x.device, dtype=x.dtype)
    y2 = None if w2 is None else torch.empty(*lead, w2.shape[0], device=x.device, dtype=x.dtype)
    nat.call("mqc_gemm_skinny_nt", x2, x2.data_ptr(), M, K, w1.data_ptr(), nat.ptr(b1),
             y1.data_ptr(), w1.shape[0], nat.ptr(w2), nat.ptr(b2), nat.ptr(y2),
             0 if w2 is None else w2.shape[0], nat.dtype_code(x2), nat.stream_of(x2))
    return y1 if w2 is None else (y1, y2)


class QuaternionLinear(nn.Module):
    def __init__(self, in_features: int, out_features: int, input_type: str = "real",
                 output_type: str = "quaternion", bias: bool = True):
        super().__init__()
        assert input_type in _KINDS
        assert output_type in _KINDS
        if input_type == "quaternion":
            assert in_features % 4 == 0, f"in_features must be divisible by 4, got {in_features}"
        if output_type == "quaternion":
            assert out_features % 4 == 0, f"out_features must be divisible by 4, got {out_features}"
        self.in_features = in_features
        self.out_features = out_features
        self.input_type = input_type
        self.output_type = output_type

        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        # Fan terms count quaternion features once (reference :96-119).
        fan_in = in_features // 4 if input_type == "quaternion" else in_features
        fan_out = out_features // 4 if output_type == "quaternion" else out_features
        if input_type == "real" and output_type == "real":
            nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        else:
            nn.init.normal_(self.weight, mean=0.0, std=math.sqrt(2.0 / (fan_in + fan_out)))

        if bias:
            shape = (out_features // 4, 4) if output_type == "quaternion" else (out_features,)
            self.bias = nn.Parameter(torch.zeros(shape))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.input_type == "quaternion":
            x = x.reshape(*x.shape[:-2], x.shape[-2] * 4)
        if self.output_type == "real":
            return F.linear(x, self.weight, self.bias)
        out = wide_linear(x, self.weight)
        out = out.view(*out.shape[:-1], self.out_features // 4, 4)
        if self.bias is not None:
            out = out + self.bias
        return out

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"input_type={self.input_type}, output_type={self.output_type}, "
                f"bias={self.bias is not None}")


class QuaternionLinearTensorCore(nn.Module):
    """Placeholder kept for API parity (reference :211-222 raises the same way)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        raise NotImplementedError("TensorCore-optimized version not yet implemented")


def real_to_quaternion_projection(in_features: int, out_quat_dim: int,
                                  bias: bool = True) -> QuaternionLinear:
    """R^in -> H^out_quat_dim. Reference: quaternion_linear.py:227-245."""
    return QuaternionLinear(in_features, out_quat_dim * 4, "real", "quaternion", bias)


def quaternion_to_real_projection(in_quat_dim: int, out_features: int,
                                  bias: bool = True) -> QuaternionLinear:
    """H^in_quat_dim -> R^out. Reference: quaternion_linear.py:248-266."""
    return QuaternionLinear(in_quat_dim * 4, out_features, "quaternion", "real", bias)
