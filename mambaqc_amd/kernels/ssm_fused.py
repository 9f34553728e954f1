"""Quaternion SSM recurrence on the GPU.

Mirrors mambaqc/kernels/ssm_fused.py (ssm_step_fused :258-337,
ssm_forward_fused :340-401):
    h_t = q_t (x) h_{t-1} + B_t (x) S_t        (S broadcast over d_state)
    y_t = sum_k C_{t,k} (x) h_{t,k} + D_t * S_t
One HIP launch walks every time step (the reference launches one kernel per
step); the state never leaves registers.

`ssm_forward_fused_dl` is the block's fused form: it takes delta and the raw
Lambda parameters instead of a materialised q, computes the Cayley
discretisation of z = delta * Lambda in registers, and takes the real
selected signal s (S = (s, 0, 0, 0)). It replaces
mambaqc/models/quaternion_mamba2_block.py:206-228.
"""
from __future__ import annotations

import torch

from .. import _native as nat


def _d_strides(D: torch.Tensor, dtype: torch.dtype):
    """Return (tensor, (sb, st, sd)) for a [B, T, D] skip tensor in `dtype`.

    An expanded [D] vector (zero batch and time strides, the block's
    D.unsqueeze(0).unsqueeze(0).expand(...)) is passed without materialising it.
    """
    sb, st, sd = D.stride()
    if sb == 0 and st == 0:
        vec = D[0, 0].to(dtype).contiguous()
        return vec, (0, 0, 1)
    D = D.to(dtype).contiguous()
    return D, tuple(D.stride())


def _launch_q(q, B, S, C, D, h0, batch, T, d_model, d_state, name, want_state):
    dtype = q.dtype
    for t in (B, S, C):
        if t.dtype != dtype:
            raise TypeError(f"{name}: dtype mismatch {dtype} vs {t.dtype}")
    q, B, S, C = (nat.aligned16(t) for t in (q, B, S, C))
    Dt, (sb, st, sd) = D
    y = torch.empty(batch, T, d_model, 4, device=q.device, dtype=dtype)
    h_last = (torch.empty(batch, d_model, d_state, 4, device=q.device, dtype=dtype)
              if want_state else None)
    if h0 is not None:
        if h0.dtype != dtype:
            raise TypeError(f"{name}: dtype mismatch {dtype} vs {h0.dtype}")
        h0 = nat.aligned16(h0)
    nat.call("mqc_ssm_q_fwd", q, q.data_ptr(), B.data_ptr(), S.data_ptr(), C.data_ptr(),
             Dt.data_ptr(), sb, st, sd, nat.ptr(h0), y.data_ptr(), nat.ptr(h_last),
             batch, T, d_model, d_state, nat.dtype_code(q), nat.stream_of(q))
    return y, h_last


def ssm_step_fused(q: torch.Tensor, B: torch.Tensor, S: torch.Tensor, C: torch.Tensor,
                   D: torch.Tensor, h_prev: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """One step. q, B, C, h_prev: [batch, d_model, d_state, 4]; S: [batch, d_model, 4];
    D: [batch, d_model]. Returns (h_new, y[batch, d_model, 4]).

    Reference: ssm_fused.py:258-337 (asserts :290-294).
    """
    batch_size, d_model, d_state, _ = q.shape
    assert B.shape == (batch_size, d_model, d_state, 4)
    assert S.shape == (batch_size, d_model, 4)
    assert C.shape == (batch_size, d_model, d_state, 4)
    assert D.shape == (batch_size, d_model)
    assert h_prev.shape == (batch_size, d_model, d_state, 4)
    nat.require_device("ssm_step_fused", q, B, S, C, D, h_prev)
    Dv = D.to(q.dtype).contiguous()
    y, h_new = _launch_q(q, B, S, C, (Dv, (Dv.stride(0), 0, Dv.stride(1))), h_prev,
                         batch_size, 1, d_model, d_state, "ssm_step_fused", True)
    return h_new, y.view(batch_size, d_model, 4)


def ssm_forward_fused(q: torch.Tensor, B: torch.Tensor, S: torch.Tensor, C: torch.Tensor,
                      D: torch.Tensor) -> torch.Tensor:
    """All time steps from a zero state.

    q, B, C: [batch, seq_len, d_model, d_state, 4]; S: [batch, seq_len, d_model, 4];
    D: [batch, seq_len, d_model] (may be an expanded view). Returns
    y: [batch, seq_len, d_model, 4] in q's dtype. Reference: ssm_fused.py:340-401.
    """
    batch_size, seq_len, d_model, d_state, _ = q.shape
    assert B.shape == q.shape and C.shape == q.shape, "B and C must match q's shape"
    assert S.shape == (batch_size, seq_len, d_model, 4)
    assert D.shape == (batch_size, seq_len, d_model)
    nat.require_device("ssm_forward_fused", q, B, S, C, D)
    y, _ = _launch_q(q, B, S, C, _d_strides(D, q.dtype), None, batch_size, seq_len, d_model,
                     d_state, "ssm_forward_fused", False)
    return y


def _dl_check(delta, s, B, C, lambda_alpha, lambda_imag, D, h0):
    batch, T, d_inner, d_state, four = B.shape
    assert four == 4
    assert C.shape == B.shape
    assert delta.shape == (batch, T, d_inner) and s.shape == (batch, T, d_inner)
    assert lambda_alpha.shape == (d_inner, d_state)
    assert lambda_imag.shape == (d_inner, d_state, 3)
    assert D.shape == (d_inner,)
    if h0 is not None:
        assert h0.shape == (batch, d_inner, d_state, 4)
    nat.require_device("ssm_forward_fused_dl", delta, s, B, C, lambda_alpha, lambda_imag, D)
    if C.dtype != B.dtype:
        raise TypeError(f"ssm_forward_fused_dl: dtype mismatch {B.dtype} vs {C.dtype}")
    return batch, T, d_inner, d_state


def _dl_operands(delta, s, B, C, lambda_alpha, lambda_imag, D, h0):
    """Contiguous, aligned operands in the kernel's types (fp32 parameters)."""
    dtype = B.dtype
    ops = [nat.aligned16(t.detach().to(dtype)) for t in (delta, s)]
    ops += [nat.aligned16(t.detach()) for t in (B, C)]
    ops += [nat.param_f32(t) for t in (lambda_alpha, lambda_imag, D)]
    # The state is fp32 at the boundary whatever the operands' dtype.
    ops.append(None if h0 is None else nat.aligned16(h0.detach().float()))
    return ops


# Largest d_state the backward kernel takes (one lane per state, a group of
# d_state lanes per (b, d) inside one wave: include/mambaqc_hip.h,
# mqc_ssm_fused_bwd). The inference walk goes to 256.
SSM_BWD_MAX_STATE = 64


def _require_trainable_state(B: torch.Tensor) -> None:
    """Refuse, before any launch or allocation, a training forward whose
    backward the library cannot run (d_state above SSM_BWD_MAX_STATE)."""
    d_state = B.shape[-2] if B.dim() >= 2 else 0
    if d_state > SSM_BWD_MAX_STATE:
        raise ValueError(
            f"ssm_forward_fused_dl: gradients need d_state <= {SSM_BWD_MAX_STATE} "
            f"(got {d_state}); run without autograd (torch.no_grad) for inference")


def train_chunk_len(batch: int, seq_len: int, d_inner: int, d_state: int,
                    dtype: torch.dtype, chunk_len: int | None = None) -> int:
    """Chunk length of the training walk and the backward: the inference
    walk's choice (chunk_len_for) or `chunk_len`, rounded up to a multiple of
    the checkpoint interval (seq_len or more: the whole walk)."""
    code = nat.dtype_code(torch.empty(0, dtype=dtype))
    K = int(nat.load().mqc_ssm_bwd_ckpt_every(code))
    if chunk_len is not None and int(chunk_len) < 1:
        raise ValueError(f"chunk_len must be >= 1, got {chunk_len}")
    if chunk_len is not None:
        return -(-int(chunk_len) // K) * K
    L = -(-chunk_len_for(batch, seq_len, d_inner, d_state, dtype) // K) * K
    # Rounding up only lowers the chunk count, so the library's bound on
    # batch * n_chunks (65535) still holds; kept explicit for the launches.
    if L < seq_len and batch * -(-seq_len // L) > 65535:
        return seq_len
    return L


def _chunk_workspace(batch, T, d_inner, d_state, L, device):
    nbytes = int(nat.load().mqc_ssm_chunked_workspace_bytes(batch, T, d_inner, d_state, L))
    if nbytes < 0:
        nat.check(nbytes, "mqc_ssm_chunked_workspace_bytes")
    return torch.empty(max(nbytes, 16), device=device, dtype=torch.uint8), nbytes


def ssm_fused_dl_train_forward(delta, s, B, C, lambda_alpha, lambda_imag, D, h0=None,
                               eps: float = 1e-6, chunk_len: int | None = None):
    """Training forward of the block's SSM: y, the final state, and what the
    backward needs (the kernel operands and the fp32 state checkpoints).

    Returns (y, h_last, saved) with saved = (delta, s, B, C, lambda_alpha,
    lambda_imag, D, h0, checkpoints) in the kernel's types. Small batches walk
    in time chunks (train_chunk_len; chunk_len forces a length).
    """
    _require_trainable_state(B)
    batch, T, d_inner, d_state = _dl_check(delta, s, B, C, lambda_alpha, lambda_imag, D, h0)
    dl, sv, Bc, Cc, la, li, Dv, h0c = _dl_operands(delta, s, B, C, lambda_alpha, lambda_imag,
                                                   D, h0)
    code = nat.dtype_code(Bc)
    K = nat.load().mqc_ssm_bwd_ckpt_every(code)
    n_ckpt = (T + K - 1) // K
    y = torch.empty(batch, T, d_inner, 4, device=Bc.device, dtype=Bc.dtype)
    h_last = torch.empty(batch, d_inner, d_state, 4, device=Bc.device, dtype=torch.float32)
    ckpt = torch.empty(batch, max(n_ckpt, 1), d_inner, d_state, 4, device=Bc.device,
                       dtype=torch.float32)
    L = train_chunk_len(batch, T, d_inner, d_state, Bc.dtype, chunk_len)
    if 0 < L < T:
        ws, nbytes = _chunk_workspace(batch, T, d_inner, d_state, L, Bc.device)
        nat.call("mqc_ssm_fused_fwd_train_chunked", Bc, dl.data_ptr(), sv.data_ptr(),
                 Bc.data_ptr(), Cc.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(),
                 nat.ptr(h0c), y.data_ptr(), h_last.data_ptr(), ckpt.data_ptr(), K, batch, T,
                 d_inner, d_state, L, float(eps), code, ws.data_ptr(), nbytes,
                 nat.stream_of(Bc))
    else:
        nat.call("mqc_ssm_fused_fwd_train", Bc, dl.data_ptr(), sv.data_ptr(), Bc.data_ptr(),
                 Cc.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(), nat.ptr(h0c),
                 y.data_ptr(), h_last.data_ptr(), ckpt.data_ptr(), K, batch, T, d_inner,
                 d_state, float(eps), code, nat.stream_of(Bc))
    return y, h_last, (dl, sv, Bc, Cc, la, li, Dv, h0c, ckpt)


def ssm_fused_dl_backward(saved, gy, gh_last=None, eps: float = 1e-6,
                          chunk_len: int | None = None):
    """Backward of ssm_fused_dl_train_forward given dL/dy (and dL/dh_last).

    Returns (d_delta, d_s fp32 [batch, T, d_inner], dB, dC in B's dtype,
    dlambda_alpha, dlambda_imag, dD fp32 (summed over the batch), dh0 or None).
    """
    dl, sv, Bc, Cc, la, li, Dv, h0c, ckpt = saved
    batch, T, d_inner, d_state, _ = Bc.shape
    dtype, dev = Bc.dtype, Bc.device
    code = nat.dtype_code(Bc)
    K = nat.load().mqc_ssm_bwd_ckpt_every(code)
    if gy is None:
        gy = torch.zeros(batch, T, d_inner, 4, device=dev, dtype=dtype)
    gy = nat.aligned16(gy.to(dtype))
    if gh_last is not None:
        gh_last = nat.aligned16(gh_last.float())
    d_delta = torch.empty(dl.shape, device=dev, dtype=torch.float32)
    d_s = torch.empty(sv.shape, device=dev, dtype=torch.float32)
    dB = torch.empty_like(Bc)
    dC = torch.empty_like(Cc)
    L = train_chunk_len(batch, T, d_inner, d_state, dtype, chunk_len)
    rows = batch * (-(-T // L)) if 0 < L < T else batch  # partials: (chunk, batch) rows
    dla = torch.empty(rows, d_inner, d_state, device=dev, dtype=torch.float32)
    dli = torch.empty(rows, d_inner, d_state, 3, device=dev, dtype=torch.float32)
    dD = torch.empty(rows, d_inner, device=dev, dtype=torch.float32)
    dh0 = torch.empty_like(h0c) if h0c is not None else None
    if 0 < L < T:
        ws, nbytes = _chunk_workspace(batch, T, d_inner, d_state, L, dev)
        nat.call("mqc_ssm_fused_bwd_chunked", Bc, dl.data_ptr(), sv.data_ptr(), Bc.data_ptr(),
                 Cc.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(), nat.ptr(h0c),
                 ckpt.data_ptr(), K, gy.data_ptr(), nat.ptr(gh_last), d_delta.data_ptr(),
                 d_s.data_ptr(), dB.data_ptr(), dC.data_ptr(), dla.data_ptr(), dli.data_ptr(),
                 dD.data_ptr(), nat.ptr(dh0), batch, T, d_inner, d_state, L, float(eps), code,
                 ws.data_ptr(), nbytes, nat.stream_of(Bc))
    else:
        nat.call("mqc_ssm_fused_bwd", Bc, dl.data_ptr(), sv.data_ptr(), Bc.data_ptr(),
                 Cc.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(), nat.ptr(h0c),
                 ckpt.data_ptr(), K, gy.data_ptr(), nat.ptr(gh_last), d_delta.data_ptr(),
                 d_s.data_ptr(), dB.data_ptr(), dC.data_ptr(), dla.data_ptr(), dli.data_ptr(),
                 dD.data_ptr(), nat.ptr(dh0), batch, T, d_inner, d_state, float(eps), code,
                 nat.stream_of(Bc))
    return d_delta, d_s, dB, dC, dla.sum(0), dli.sum(0), dD.sum(0), dh0


class _SsmFusedDL(torch.autograd.Function):
    """Autograd wrapper: training forward (state checkpoints) + HIP backward."""

    @staticmethod
    def forward(ctx, delta, s, B, C, lambda_alpha, lambda_imag, D, h0, eps):
        y, h_last, saved = ssm_fused_dl_train_forward(delta, s, B, C, lambda_alpha,
                                                      lambda_imag, D, h0, eps)
        ctx.save_for_backward(*[t for t in saved if t is not None])
        ctx.has_h0 = h0 is not None
        ctx.meta = (eps, delta.dtype, s.dtype, lambda_alpha.dtype, lambda_imag.dtype,
                    D.dtype, None if h0 is None else h0.dtype)
        return y, h_last

    @staticmethod
    def backward(ctx, gy, gh_last):
        saved = list(ctx.saved_tensors)
        if not ctx.has_h0:
            saved.insert(7, None)
        eps, t_delta, t_s, t_la, t_li, t_D, t_h0 = ctx.meta
        d_delta, d_s, dB, dC, dla, dli, dD, dh0 = ssm_fused_dl_backward(saved, gy, gh_last, eps)
        return (d_delta.to(t_delta), d_s.to(t_s), dB, dC, dla.to(t_la), dli.to(t_li),
                dD.to(t_D), None if dh0 is None else dh0.to(t_h0), None)


def chunk_len_for(batch: int, seq_len: int, d_inner: int, d_state: int,
                  dtype: torch.dtype) -> int:
    """The chunk length the library picks for the inference walk at these sizes
    (seq_len: no chunking, the whole walk)."""
    code = nat.dtype_code(torch.empty(0, dtype=dtype))
    L = int(nat.load().mqc_ssm_chunk_len_auto(batch, seq_len, d_inner, d_state, code))
    if L < 0:
        nat.check(L, "mqc_ssm_chunk_len_auto")
    return L


def _launch_dl_inference(dl, sv, Bc, Cc, la, li, Dv, h0c, eps, return_state, chunk_len):
    batch, T, d_inner, d_state, _ = Bc.shape
    dtype, dev = Bc.dtype, Bc.device
    y = torch.empty(batch, T, d_inner, 4, device=dev, dtype=dtype)
    h_last = (torch.empty(batch, d_inner, d_state, 4, device=dev, dtype=torch.float32)
              if return_state else None)
    code = nat.dtype_code(Bc)
    if chunk_len is not None and int(chunk_len) < 1:
        raise ValueError(f"ssm_forward_fused_dl: chunk_len must be >= 1, got {chunk_len}")
    L = chunk_len_for(batch, T, d_inner, d_state, dtype) if chunk_len is None else int(chunk_len)
    if 0 < L < T:
        nbytes = int(nat.load().mqc_ssm_chunked_workspace_bytes(batch, T, d_inner, d_state, L))
        if nbytes < 0:
            nat.check(nbytes, "mqc_ssm_chunked_workspace_bytes")
        ws = torch.empty(max(nbytes, 16), device=dev, dtype=torch.uint8)
        nat.call("mqc_ssm_fused_fwd_chunked", Bc, dl.data_ptr(), sv.data_ptr(), Bc.data_ptr(),
                 Cc.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(), nat.ptr(h0c),
                 y.data_ptr(), nat.ptr(h_last), batch, T, d_inner, d_state, L, float(eps), code,
                 ws.data_ptr(), nbytes, nat.stream_of(Bc))
    else:
        nat.call("mqc_ssm_fused_fwd", Bc, dl.data_ptr(), sv.data_ptr(), Bc.data_ptr(),
                 Cc.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(), nat.ptr(h0c),
                 y.data_ptr(), nat.ptr(h_last), batch, T, d_inner, d_state, float(eps), code,
                 nat.stream_of(Bc))
    return (y, h_last) if return_state else y


def ssm_forward_fused_dl(delta: torch.Tensor, s: torch.Tensor, B: torch.Tensor,
                         C: torch.Tensor, lambda_alpha: torch.Tensor,
                         lambda_imag: torch.Tensor, D: torch.Tensor, eps: float = 1e-6,
                         h0: torch.Tensor | None = None, return_state: bool = False,
                         chunk_len: int | None = None):
    """The block's SSM with the Cayley discretisation fused in.

    delta, s: [batch, seq_len, d_inner]; B, C: [batch, seq_len, d_inner, d_state, 4];
    lambda_alpha: [d_inner, d_state]; lambda_imag: [d_inner, d_state, 3]; D: [d_inner];
    h0: optional [batch, d_inner, d_state, 4] initial state.
    Computes Lambda = (-softplus(lambda_alpha), tanh(lambda_imag)),
    q_t = Cayley(delta_t * Lambda, eps), and the recurrence with S = (s, 0, 0, 0).
    Returns y [batch, seq_len, d_inner, 4] in B's dtype (and the final state,
    fp32 [batch, d_inner, d_state, 4], if return_state). The state is carried in
    fp32 across calls as within one, so feeding a sequence in pieces from the
    returned state gives the whole sequence's y.

    Differentiable in every tensor argument when autograd is recording (HIP
    backward, d_state <= 64). Otherwise one inference walk: whole, or, for
    batches too small to fill the GPU, cut into chunks of `chunk_len` steps
    walked side by side (None: the library's choice, chunk_len_for; an int
    forces that length, >= seq_len meaning the whole walk).
    """
    inputs = (delta, s, B, C, lambda_alpha, lambda_imag, D) + ((h0,) if h0 is not None else ())
    if nat.compiling():
        return _dl_ops(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, eps, return_state,
                       chunk_len, inputs)
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
        _require_trainable_state(B)
        y, h_last = _SsmFusedDL.apply(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, eps)
        return (y, h_last) if return_state else y
    _dl_check(delta, s, B, C, lambda_alpha, lambda_imag, D, h0)
    ops = _dl_operands(delta, s, B, C, lambda_alpha, lambda_imag, D, h0)
    return _launch_dl_inference(*ops, eps, return_state, chunk_len)


def _dl_ops(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, eps, return_state, chunk_len,
            inputs):
    """The delta-lambda SSM through the registered operators (torch.compile):
    the training walk when autograd records, else the inference walk."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
        _require_trainable_state(B)
        y, h_last, _ = torch.ops.mambaqc.ssm_forward_dl_train(delta, s, B, C, lambda_alpha,
                                                              lambda_imag, D, h0, eps)
    else:
        y, h_last = torch.ops.mambaqc.ssm_forward_dl(delta, s, B, C, lambda_alpha, lambda_imag,
                                                     D, h0, eps, chunk_len)
    return (y, h_last) if return_state else y


def ssm_forward_front_dl_state_(dt_raw: torch.Tensor, g_raw: torch.Tensor, x: torch.Tensor,
                                B: torch.Tensor, C: torch.Tensor, lambda_alpha: torch.Tensor,
                                lambda_imag: torch.Tensor, D: torch.Tensor, h: torch.Tensor,
                                eps: float = 1e-6) -> torch.Tensor:
    """ssm_forward_front_dl continued from the state h, which is overwritten
    with the final state; returns y. For the recurrent decode step (no autograd):
    h is fp32 [batch, d_inner, d_state, 4], contiguous, and is both the kernel's
    h0 and its h_last (one whole walk, in which each state is written only by the
    lane that read it)."""
    if torch.is_grad_enabled() and any(
            t.requires_grad for t in (dt_raw, g_raw, x, B, C, lambda_alpha, lambda_imag, D, h)):
        raise RuntimeError("ssm_forward_front_dl_state_: updates its state in place; "
                           "run under torch.no_grad")
    if h.dtype != torch.float32 or not h.is_contiguous() or h.data_ptr() % 16:
        raise ValueError("ssm_forward_front_dl_state_: h must be a contiguous, 16-byte "
                         "aligned fp32 [batch, d_inner, d_state, 4] tensor")
    delta, s = ssm_front(dt_raw, g_raw, x)
    batch, T, d_inner, d_state = _dl_check(delta, s, B, C, lambda_alpha, lambda_imag, D, h)
    dl, sv, Bc, Cc, la, li, Dv, _ = _dl_operands(delta, s, B, C, lambda_alpha, lambda_imag, D,
                                                 None)
    y = torch.empty(batch, T, d_inner, 4, device=Bc.device, dtype=Bc.dtype)
    nat.call("mqc_ssm_fused_fwd", Bc, dl.data_ptr(), sv.data_ptr(), Bc.data_ptr(), Cc.data_ptr(),
             la.data_ptr(), li.data_ptr(), Dv.data_ptr(), h.data_ptr(), y.data_ptr(),
             h.data_ptr(), batch, T, d_inner, d_state, float(eps), nat.dtype_code(Bc),
             nat.stream_of(Bc))
    return y


def _front_operands(dt_raw, g_raw, x):
    if not (dt_raw.shape == g_raw.shape == x.shape):
        raise ValueError(f"ssm_front: shapes differ {tuple(dt_raw.shape)}, "
                         f"{tuple(g_raw.shape)}, {tuple(x.shape)}")
    nat.require_device("ssm_front", dt_raw, g_raw, x)
    ct = torch.promote_types(torch.promote_types(dt_raw.dtype, g_raw.dtype), x.dtype)
    return [nat.aligned16(t.detach().to(ct)) for t in (dt_raw, g_raw, x)]


def _front_forward(dt, g, xv):
    delta = torch.empty_like(dt)
    s = torch.empty_like(dt)
    nat.call("mqc_ssm_front_fwd", dt, dt.data_ptr(), g.data_ptr(), xv.data_ptr(),
             delta.data_ptr(), s.data_ptr(), dt.numel(), nat.dtype_code(dt), nat.stream_of(dt))
    return delta, s


def ssm_front(dt_raw: torch.Tensor, g_raw: torch.Tensor, x: torch.Tensor):
    """delta = softplus(dt_raw), s = sigmoid(g_raw) * x in one HIP pass (inference).

    dt_raw is dt_proj's output and g_raw gate_proj's, as in
    mambaqc/models/quaternion_mamba2_block.py:183,197-198. The three tensors have
    one shape; the results come in their promoted dtype (fp32 arithmetic).
    """
    if nat.compiling():
        return torch.ops.mambaqc.ssm_front(dt_raw, g_raw, x)
    return _front_forward(*_front_operands(dt_raw, g_raw, x))


def _front_backward(dt, g, xv, d_delta, d_s):
    d_dt, d_g, d_x = (torch.empty_like(dt) for _ in range(3))
    d_delta = nat.aligned16(d_delta.float())
    d_s = nat.aligned16(d_s.float())
    nat.call("mqc_ssm_front_bwd", dt, dt.data_ptr(), g.data_ptr(), xv.data_ptr(),
             d_delta.data_ptr(), d_s.data_ptr(), d_dt.data_ptr(), d_g.data_ptr(),
             d_x.data_ptr(), dt.numel(), nat.dtype_code(dt), nat.stream_of(dt))
    return d_dt, d_g, d_x


class _SsmFrontFusedDL(torch.autograd.Function):
    """Front (softplus / sigmoid gate) + SSM as one autograd node, so the SSM's
    fp32 d_delta and d_s reach the front's backward without a round trip
    through the (possibly fp16) dtype of delta and s."""

    @staticmethod
    def forward(ctx, dt_raw, g_raw, x, B, C, lambda_alpha, lambda_imag, D, h0, eps):
        dt, g, xv = _front_operands(dt_raw, g_raw, x)
        delta, s = _front_forward(dt, g, xv)
        y, h_last, saved = ssm_fused_dl_train_forward(delta, s, B, C, lambda_alpha,
                                                      lambda_imag, D, h0, eps)
        del delta, s
        ctx.save_for_backward(dt, g, xv, *[t for t in saved if t is not None])
        ctx.has_h0 = h0 is not None
        ctx.meta = (eps, dt_raw.dtype, g_raw.dtype, x.dtype, lambda_alpha.dtype,
                    lambda_imag.dtype, D.dtype, None if h0 is None else h0.dtype)
        return y, h_last

    @staticmethod
    def backward(ctx, gy, gh_last):
        dt, g, xv, *saved = ctx.saved_tensors
        if not ctx.has_h0:
            saved.insert(7, None)
        eps, t_dt, t_g, t_x, t_la, t_li, t_D, t_h0 = ctx.meta
        d_delta, d_s, dB, dC, dla, dli, dD, dh0 = ssm_fused_dl_backward(saved, gy, gh_last, eps)
        d_dt, d_g, d_x = _front_backward(dt, g, xv, d_delta, d_s)
        return (d_dt.to(t_dt), d_g.to(t_g), d_x.to(t_x), dB, dC, dla.to(t_la), dli.to(t_li),
                dD.to(t_D), None if dh0 is None else dh0.to(t_h0), None)


def ssm_forward_front_dl(dt_raw: torch.Tensor, g_raw: torch.Tensor, x: torch.Tensor,
                         B: torch.Tensor, C: torch.Tensor, lambda_alpha: torch.Tensor,
                         lambda_imag: torch.Tensor, D: torch.Tensor, eps: float = 1e-6,
                         h0: torch.Tensor | None = None, return_state: bool = False):
    """The block's whole SSM from the projections' outputs: delta =
    softplus(dt_raw), s = sigmoid(g_raw) * x, then ssm_forward_fused_dl.
    Differentiable in every tensor argument when autograd is recording."""
    inputs = (dt_raw, g_raw, x, B, C, lambda_alpha, lambda_imag, D) + (
        (h0,) if h0 is not None else ())
    if nat.compiling():
        if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
            # Front and training walk as one traced operator, whose backward
            # hands d_delta and d_s to the front in fp32 (as _SsmFrontFusedDL).
            _require_trainable_state(B)
            y, h_last, _ = torch.ops.mambaqc.ssm_front_forward_dl_train(
                dt_raw, g_raw, x, B, C, lambda_alpha, lambda_imag, D, h0, eps)
            return (y, h_last) if return_state else y
        delta, s = torch.ops.mambaqc.ssm_front(dt_raw, g_raw, x)
        return _dl_ops(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, eps, return_state,
                       None, inputs)
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
        _require_trainable_state(B)
        y, h_last = _SsmFrontFusedDL.apply(dt_raw, g_raw, x, B, C, lambda_alpha, lambda_imag,
                                           D, h0, eps)
        return (y, h_last) if return_state else y
    delta, s = ssm_front(dt_raw, g_raw, x)
    return ssm_forward_fused_dl(delta, s, B, C, lambda_alpha, lambda_imag, D, eps=eps, h0=h0,
                                return_state=return_state)


# --- B/C projections fused with the walk (inference) ---------------------------

# Batches up to this size run the fused walk with each half of the states in a
# workgroup of its own (mqc_ssm_fused_bc_fwd_split). A workgroup streams its d's weight
# rows once per 256-token tile; the workgroups of a d's batches share those reads in L2,
# a single sequence's do not, and its resident d's then want more weight rows than the
# Infinity Cache holds. Config-3 width, one call: d_state 64 at batch 1, T2048 5.26 ms in
# one workgroup per d, against 2 x 2.21 ms for two halves' worth of work (d_state 32).
FUSED_BC_SPLIT_MAX_BATCH = 1
# The split form's workspace (two fp32 partial sums of y, 49 KiB per token at d_inner
# 1536) stays under this many bytes: a longer sequence of one batch row is walked in
# segments of time, the state carried from one to the next through h0 / h_last.
FUSED_BC_SPLIT_WS_MAX = 4 << 30

def fused_bc_eligible(x: torch.Tensor, B_weight: torch.Tensor, C_weight: torch.Tensor,
                      d_state: int, dtype: torch.dtype | None = None) -> bool:
    """Whether ssm_forward_fused_bc takes these operands: x [batch, T, d_inner] with
    d_inner a multiple of 64 and weights [d_inner * d_state * 4, d_inner] of one shape,
    all bf16 or all fp16, d_state even and at most 64, all on a ROCm device. dtype:
    the type all three will be cast to first (autocast's), or None to take their own."""
    if x.dim() != 3 or not (x.is_cuda and B_weight.is_cuda and C_weight.is_cuda):
        return False
    d_inner = x.shape[-1]
    dts = (x.dtype, B_weight.dtype, C_weight.dtype) if dtype is None else (dtype,) * 3
    return (dts[0] == dts[1] == dts[2]
            and dts[0] in (torch.bfloat16, torch.float16)
            and d_inner % 64 == 0 and 0 < d_state <= 64 and d_state % 2 == 0
            and tuple(B_weight.shape) == tuple(C_weight.shape) == (d_inner * d_state * 4, d_inner))


def ssm_forward_fused_bc(x: torch.Tensor, B_weight: torch.Tensor, C_weight: torch.Tensor,
                         delta: torch.Tensor, s: torch.Tensor, lambda_alpha: torch.Tensor,
                         lambda_imag: torch.Tensor, D: torch.Tensor, eps: float = 1e-6,
                         h0: torch.Tensor | None = None, return_state: bool = False,
                         split: bool | None = None):
    """The block's B/C projections and its SSM in one HIP launch (inference, bf16 or
    fp16).

    B = x B_weight^T and C = x C_weight^T, as [batch, seq_len, d_inner, d_state, 4]
    (the bias-free real -> quaternion projections,
    mambaqc/layers/quaternion_linear.py:145-161), are computed 256 tokens at a time
    on chip, rounded to x's dtype as the projections would store them, and walked
    there by ssm_forward_fused_dl's recurrence; neither is ever written to memory.
    x: [batch, seq_len, d_inner] bf16 or fp16 (the projections' input); B_weight,
    C_weight: [d_inner * d_state * 4, d_inner] in x's dtype; delta, s (taken in x's
    dtype), the Lambda parameters, D and h0 as in ssm_forward_fused_dl. Returns y
    [batch, seq_len, d_inner, 4] in x's dtype (and the final fp32 state if
    return_state). Inference only (no autograd).
    split: run each half of the states (32) in a workgroup of its own, with a
    workspace for the halves' partial sums and a second launch adding them (the
    same y bit for bit); None splits batches of at most FUSED_BC_SPLIT_MAX_BATCH.
    """
    batch, T, d_inner = x.shape
    d_state = lambda_alpha.shape[-1] if lambda_alpha.dim() == 2 else 0
    if nat.compiling():
        y, h_last = torch.ops.mambaqc.ssm_forward_fused_bc(x, B_weight, C_weight, delta, s,
                                                           lambda_alpha, lambda_imag, D, h0, eps)
        return (y, h_last) if return_state else y
    assert delta.shape == (batch, T, d_inner) and s.shape == (batch, T, d_inner)
    assert lambda_alpha.shape == (d_inner, d_state)
    assert lambda_imag.shape == (d_inner, d_state, 3)
    assert D.shape == (d_inner,)
    if h0 is not None:
        assert h0.shape == (batch, d_inner, d_state, 4)
    nat.require_device("ssm_forward_fused_bc", x, B_weight, C_weight, delta, s, lambda_alpha,
                       lambda_imag, D)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (
            x, B_weight, C_weight, delta, s, lambda_alpha, lambda_imag, D)):
        raise RuntimeError("ssm_forward_fused_bc: inference only; run under torch.no_grad")
    if not fused_bc_eligible(x, B_weight, C_weight, d_state):
        raise ValueError("ssm_forward_fused_bc: needs bf16 or fp16 x [batch, T, d_inner] with "
                         "d_inner a multiple of 64, weights [d_inner * d_state * 4, d_inner] of "
                         "x's dtype and an even d_state <= 64")
    dt = x.dtype
    xc, wb, wc = (nat.aligned16(t.detach()) for t in (x, B_weight, C_weight))
    dl, sv = (nat.aligned16(t.detach().to(dt)) for t in (delta, s))
    la, li, Dv = (nat.param_f32(t) for t in (lambda_alpha, lambda_imag, D))
    h0c = None if h0 is None else nat.aligned16(h0.detach().float())
    y = torch.empty(batch, T, d_inner, 4, device=x.device, dtype=dt)
    code = nat.dtype_code(xc)
    h_last = (torch.empty(batch, d_inner, d_state, 4, device=x.device, dtype=torch.float32)
              if return_state else None)
    if split is None:
        split = batch <= FUSED_BC_SPLIT_MAX_BATCH
    lib = nat.load()
    ws_bytes = lib.mqc_ssm_fused_bc_split_workspace_bytes(batch, T, d_inner, d_state) if split else 0
    stream = nat.stream_of(xc)
    if ws_bytes <= 0:
        nat.call("mqc_ssm_fused_bc_fwd", xc, xc.data_ptr(), wb.data_ptr(), wc.data_ptr(),
                 dl.data_ptr(), sv.data_ptr(), la.data_ptr(), li.data_ptr(), Dv.data_ptr(),
                 nat.ptr(h0c), y.data_ptr(), nat.ptr(h_last), batch, T, d_inner, d_state,
                 float(eps), code, stream)
        return (y, h_last) if return_state else y
    # Split: one launch over the whole sequence, or (a batch of one whose workspace
    # would pass FUSED_BC_SPLIT_WS_MAX) segments of whole 256-token tiles.
    seg = T
    if batch == 1 and ws_bytes > FUSED_BC_SPLIT_WS_MAX:
        # Equal segments (whole tiles) of at most the budget's tokens.
        per_token = ws_bytes // T
        seg_max = max(256, FUSED_BC_SPLIT_WS_MAX // per_token // 256 * 256)
        n_seg = -(-T // seg_max)
        seg = -(-T // (n_seg * 256)) * 256
    if seg < T:
        ws_bytes = lib.mqc_ssm_fused_bc_split_workspace_bytes(batch, seg, d_inner, d_state)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    state = h_last
    if seg < T and state is None:
        state = torch.empty(batch, d_inner, d_state, 4, device=x.device, dtype=torch.float32)
    for t0 in range(0, T, seg):
        t1 = min(T, t0 + seg)
        # (A batch of one: every time slice is contiguous.)
        nat.call("mqc_ssm_fused_bc_fwd_split", xc, xc[:, t0:t1].data_ptr(), wb.data_ptr(),
                 wc.data_ptr(), dl[:, t0:t1].data_ptr(), sv[:, t0:t1].data_ptr(),
                 la.data_ptr(), li.data_ptr(), Dv.data_ptr(),
                 nat.ptr(h0c) if t0 == 0 else state.data_ptr(), y[:, t0:t1].data_ptr(),
                 nat.ptr(state), batch, t1 - t0, d_inner, d_state, float(eps), code,
                 ws.data_ptr(), ws_bytes, stream)
    return (y, h_last) if return_state else y

