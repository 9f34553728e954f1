"""Host-side tests that need no GPU: the C-ABI library loads and exports every
symbol include/mambaqc_hip.h declares, argument validation answers before any
HIP call, the Python mirror keeps the reference's assertions and refuses CPU
tensors, the block's parameters match the reference's seeded constructor, and
the product package never reaches the oracle.
"""
import ctypes
import hashlib
import json
import re

import pytest
import torch

from conftest import GOLDEN, ROOT

import mambaqc_amd
from mambaqc_amd import _native as nat
from mambaqc_amd import kernels as K

HEADER = ROOT / "include" / "mambaqc_hip.h"
FAKE = ctypes.c_void_p(4096)  # never dereferenced: validation fails first


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int)\s+(mqc_\w+)\(", text, re.M)))


def test_header_declares_the_api():
    names = declared_symbols()
    assert len(names) == 37, names
    assert set(nat.SIGNATURES) | set(nat.SIGNATURES_I64) <= set(names)


def test_library_exports_every_declared_symbol():
    lib = nat.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.mqc_abi_version() == nat.ABI_VERSION == 8


def test_status_strings():
    assert nat.status_string(0) == "ok"
    for code in (-1, -2, -3, -4, -5, -6, -7):
        s = nat.status_string(code)
        assert s and s != "unknown status"


def test_validation_codes_without_gpu():
    lib = nat.load()
    # NULL pointer with work to do.
    assert lib.mqc_quaternion_multiply(None, None, None, 10, 0, None) == -1
    # Negative size.
    assert lib.mqc_cayley_fwd(FAKE, FAKE, -1, 1e-6, 0, None) == -2
    # Unknown dtype.
    assert lib.mqc_quaternion_conjugate(FAKE, FAKE, 8, 7, None) == -3
    assert lib.mqc_ssm_fused_fwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, None,
                                 1, 1, 1, 1, 1e-6, 9, None) == -3
    # Misaligned quaternion pointer.
    assert lib.mqc_cumprod_scan_fwd(ctypes.c_void_p(4097), FAKE, 1, 1, 1, 0, None) == -4
    # d_state beyond the supported maximum.
    assert lib.mqc_ssm_fused_fwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, None,
                                 1, 1, 1, 300, 1e-6, 1, None) == -5
    assert lib.mqc_ssm_q_fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 1, None, FAKE, None,
                             1, 1, 1, 257, 0, None) == -5
    # QLN over an empty row is undefined (mean of nothing).
    assert lib.mqc_qln_fwd(FAKE, FAKE, FAKE, FAKE, None, None, 3, 0, 1e-5, 0, None) == -2
    # Gate row stride shorter than the row.
    assert lib.mqc_out_gate_fwd(FAKE, FAKE, 4, FAKE, FAKE, 2, 8, 0, None) == -2
    # Front of the SSM: negative size, missing output, unknown dtype, misaligned.
    assert lib.mqc_ssm_front_fwd(FAKE, FAKE, FAKE, FAKE, FAKE, -1, 0, None) == -2
    assert lib.mqc_ssm_front_fwd(FAKE, FAKE, FAKE, FAKE, None, 8, 0, None) == -1
    assert lib.mqc_ssm_front_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 4,
                                 None) == -3
    assert lib.mqc_ssm_front_fwd(ctypes.c_void_p(4097), FAKE, FAKE, FAKE, FAKE, 3, 1,
                                 None) == -4
    # Nothing to do is not an error.
    assert lib.mqc_ssm_front_bwd(None, None, None, None, None, None, None, None, 0, 1,
                                 None) == 0
    assert lib.mqc_quaternion_multiply(None, None, None, 0, 0, None) == 0
    assert lib.mqc_cumprod_scan_fwd(None, None, 0, 5, 5, 0, None) == 0


def test_wrappers_keep_reference_assertions():
    # Shape assertions fire before the device check, as in the reference.
    with pytest.raises(AssertionError):
        K.quaternion_multiply(torch.zeros(3, 4), torch.zeros(2, 4))
    with pytest.raises(AssertionError):
        K.cayley_discretization_fused(torch.zeros(2, 3, 4))
    with pytest.raises(AssertionError):
        K.parallel_scan_quaternion(torch.zeros(1, 2, 3, 4, 3))
    with pytest.raises(AssertionError):
        K.quaternion_layer_norm_fused(torch.zeros(1, 2, 3, 4), torch.ones(4), torch.zeros(3, 4))
    with pytest.raises(AssertionError):
        K.ssm_step_fused(torch.zeros(1, 2, 3, 4), torch.zeros(1, 2, 3, 4), torch.zeros(1, 2, 4),
                         torch.zeros(1, 2, 3, 4), torch.zeros(1, 3), torch.zeros(1, 2, 3, 4))


def test_wrappers_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match="ROCm device"):
        K.quaternion_multiply(torch.zeros(3, 4), torch.zeros(3, 4))
    with pytest.raises(RuntimeError, match="ROCm device"):
        K.cayley_discretization_fused(torch.zeros(1, 2, 3, 4, 4))
    with pytest.raises(RuntimeError, match="ROCm device"):
        K.QuaternionLayerNorm(3)(torch.zeros(1, 2, 3, 4))


def test_block_training_forward_refuses_cpu():
    blk = mambaqc_amd.QuaternionMamba2Block(8, d_state=2)
    with pytest.raises(RuntimeError, match="ROCm device"):
        blk(torch.zeros(1, 3, 8))


def test_training_forward_refuses_d_state_above_backward_limit():
    """A recorded forward with d_state > 64 fails at once with a clear error
    (before any launch or allocation), not inside backward after the whole
    training forward has run; d_state 64 passes the check and reaches the
    device check."""
    from mambaqc_amd.kernels.ssm_fused import SSM_BWD_MAX_STATE

    assert SSM_BWD_MAX_STATE == 64
    for fn, lead in ((K.ssm_forward_fused_dl, 2), (K.ssm_forward_front_dl, 3)):
        for d_state, err in ((65, ValueError), (64, RuntimeError)):
            b, t, d = 1, 3, 2
            args = [torch.zeros(b, t, d, requires_grad=True) for _ in range(lead)]
            args += [torch.zeros(b, t, d, d_state, 4), torch.zeros(b, t, d, d_state, 4),
                     torch.zeros(d, d_state), torch.zeros(d, d_state, 3), torch.zeros(d)]
            with pytest.raises(err, match="d_state <= 64" if err is ValueError else "ROCm"):
                fn(*args)


def test_training_validation_codes_without_gpu():
    lib = nat.load()
    assert lib.mqc_ssm_bwd_ckpt_every(0) == 4
    assert lib.mqc_ssm_bwd_ckpt_every(1) == 8
    assert lib.mqc_ssm_bwd_ckpt_every(2) == 8
    assert lib.mqc_ssm_bwd_ckpt_every(5) == -3
    P = [FAKE] * 7
    # Checkpoint interval below 1.
    assert lib.mqc_ssm_fused_fwd_train(*P, None, FAKE, None, FAKE, 0, 1, 4, 2, 8,
                                       1e-6, 1, None) == -2
    # Missing checkpoint buffer.
    assert lib.mqc_ssm_fused_fwd_train(*P, None, FAKE, None, None, 8, 1, 4, 2, 8,
                                       1e-6, 1, None) == -1
    # Backward: interval other than the one the kernel needs, then d_state > 64.
    G = [FAKE] * 7
    assert lib.mqc_ssm_fused_bwd(*P, None, FAKE, 5, FAKE, None, *G, None, 1, 4, 2, 8,
                                 1e-6, 1, None) == -5
    assert lib.mqc_ssm_fused_bwd(*P, None, FAKE, 8, FAKE, None, *G, None, 1, 4, 2, 65,
                                 1e-6, 1, None) == -5
    # QLN backward: empty rows are an error, nothing to do is not.
    assert lib.mqc_qln_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 3, 0, 1e-5, 0, None) == -2
    assert lib.mqc_qln_bwd(None, None, None, None, None, None, None, 0, 4, 1e-5, 0, None) == 0
    # Gate backward: dz narrower than the gated columns.
    assert lib.mqc_out_gate_bwd(FAKE, FAKE, 8, FAKE, FAKE, FAKE, 2, 8, 4, 0, None) == -2


def test_chunk_policy_and_workspace_without_gpu():
    """The library's chunk choice for the inference walk: none where
    batch * d_inner * d_state states come near filling the GPU (config 3's
    393 216 states, or half of them) or the walk is short; chunks of at least
    64 steps, more for fewer states (states x chunks about 393 216), at most
    1024 of them.
    The workspace size formula, and the chunked entry point's validation."""
    from mambaqc_amd.kernels.ssm_fused import chunk_len_for

    bf = torch.bfloat16
    assert chunk_len_for(4, 2048, 1536, 64, bf) == 2048
    assert chunk_len_for(1, 100, 1536, 64, bf) == 100
    assert chunk_len_for(1, 2048, 1536, 128, bf) == 2048  # d_state > 64: whole walk
    L = chunk_len_for(1, 2048, 1536, 64, bf)
    assert 64 <= L < 2048 and -(-2048 // L) <= 8
    # Measured slower with chunks: batch 2, and d_state 16 at batch 4.
    assert chunk_len_for(2, 2048, 1536, 64, bf) == 2048
    assert chunk_len_for(4, 2048, 1536, 16, bf) == 2048
    L8 = chunk_len_for(1, 2048, 768, 64, bf)
    assert 64 <= L8 < L and -(-2048 // L8) <= 8
    # Long walks of few states: chunks until states x chunks reaches 393 216.
    assert chunk_len_for(1, 262144, 8, 64, bf) == -(-262144 // 768)
    assert chunk_len_for(1, 16384, 96, 64, bf) == 256
    assert chunk_len_for(1, 1 << 20, 1, 64, bf) == 1024  # 1024 chunks at most
    assert chunk_len_for(1, 2048, 8, 64, bf) == 64        # chunks of 64 steps at least
    lib = nat.load()
    assert lib.mqc_ssm_chunked_workspace_bytes(1, 2048, 1536, 64, 512) == 24 * 3 * 1536 * 64
    assert lib.mqc_ssm_chunked_workspace_bytes(2, 10, 3, 4, 10) == 0
    assert lib.mqc_ssm_chunked_workspace_bytes(2, 10, 3, 4, 0) == -2
    assert lib.mqc_ssm_chunk_len_auto(1, 8, 1, 1, 9) == -3
    P = [FAKE] * 7
    need = lib.mqc_ssm_chunked_workspace_bytes(1, 100, 4, 8, 10)
    # chunk_len 0; workspace missing, too small; d_state above the chunked limit.
    assert lib.mqc_ssm_fused_fwd_chunked(*P, None, FAKE, None, 1, 100, 4, 8, 0, 1e-6, 1,
                                         FAKE, need, None) == -2
    assert lib.mqc_ssm_fused_fwd_chunked(*P, None, FAKE, None, 1, 100, 4, 8, 10, 1e-6, 1,
                                         None, need, None) == -1
    assert lib.mqc_ssm_fused_fwd_chunked(*P, None, FAKE, None, 1, 100, 4, 8, 10, 1e-6, 1,
                                         FAKE, need - 1, None) == -6
    assert lib.mqc_ssm_fused_fwd_chunked(*P, None, FAKE, None, 1, 100, 4, 65, 10, 1e-6, 1,
                                         FAKE, 1 << 40, None) == -5


def test_chunked_walks_refuse_in_place_state_without_gpu():
    """With more than one chunk, chunk 0 reads h0 while the last chunk writes
    h_last in the same launch: the chunked entry points refuse overlapping
    state buffers (MQC_E_OVERLAP) before any HIP call; the whole walk (one
    chunk) keeps taking h_last == h0."""
    lib = nat.load()
    P = [FAKE] * 7
    b, T, d, k, L = 1, 100, 4, 8, 10
    nbytes = b * d * k * 16
    need = lib.mqc_ssm_chunked_workspace_bytes(b, T, d, k, L)
    H = ctypes.c_void_p(1 << 20)
    H_part = ctypes.c_void_p((1 << 20) + nbytes - 16)
    H_next = ctypes.c_void_p((1 << 20) + nbytes)
    for h_last in (H, H_part):
        assert lib.mqc_ssm_fused_fwd_chunked(*P, H, FAKE, h_last, b, T, d, k, L, 1e-6, 1,
                                             FAKE, need, None) == -7
        assert lib.mqc_ssm_fused_fwd_chunked_noalloc(*P, H, FAKE, h_last, b, T, d, k, L,
                                                     1e-6, 1, None) == -7
    # Adjacent buffers pass this check and fail the next one (no workspace).
    assert lib.mqc_ssm_fused_fwd_chunked(*P, H, FAKE, H_next, b, T, d, k, L, 1e-6, 1,
                                         None, need, None) == -1
    K = lib.mqc_ssm_bwd_ckpt_every(1)
    Lk = K * 2
    need_k = lib.mqc_ssm_chunked_workspace_bytes(b, T, d, k, Lk)
    assert lib.mqc_ssm_fused_fwd_train_chunked(*P, H, FAKE, H, FAKE, K, b, T, d, k, Lk, 1e-6,
                                               1, FAKE, need_k, None) == -7
    G = [FAKE] * 7
    # dh_last (the 11th argument) and dh0 (the 20th) overlapping.
    assert lib.mqc_ssm_fused_bwd_chunked(*P, None, FAKE, K, FAKE, H, *G[:4], FAKE, FAKE, FAKE,
                                         H, b, T, d, k, Lk, 1e-6, 1, FAKE, need_k, None) == -7


def test_whole_walks_refuse_shifted_state_alias_without_gpu():
    """The whole walks and the fused B/C walk take h_last == h0, but refuse state
    buffers that share bytes without being the same buffer (one lane could then
    overwrite another's h0 before it is read): MQC_E_OVERLAP before any HIP call."""
    lib = nat.load()
    b, T, d, k = 1, 100, 64, 8
    nbytes = b * d * k * 16
    H = ctypes.c_void_p(1 << 20)
    H_part = ctypes.c_void_p((1 << 20) + nbytes - 16)
    # (delta, s, B, C, lambda_alpha, lambda_imag, D, h0, y, h_last, b, T, d, k, eps, dtype, stream)
    assert lib.mqc_ssm_fused_fwd(*[FAKE] * 7, H, FAKE, H_part, b, T, d, k, 1e-6, 1, None) == -7
    # (q, B, S, C, D, d_sb, d_st, d_sd, h0, y, h_last, b, T, d, k, dtype, stream): bf16
    # state, 8 bytes per quaternion.
    H_half = ctypes.c_void_p((1 << 20) + nbytes // 2 - 8)
    assert lib.mqc_ssm_q_fwd(*[FAKE] * 5, 0, 0, 0, H, FAKE, H_half, b, T, d, k, 1, None) == -7
    # (x, W_B, W_C, delta, s, lambda_alpha, lambda_imag, D, h0, y, h_last, b, T, d, k, eps,
    #  dtype, stream)
    assert lib.mqc_ssm_fused_bc_fwd(*[FAKE] * 8, H, FAKE, H_part, b, T, d, k, 1e-6, 1,
                                    None) == -7


def test_out_proj_gate_refuses_overlap_without_gpu():
    """The fused output step writes out tile by tile while other tiles still read
    y, W, bias and z: out sharing bytes with any of them, or with x without being
    x, is refused (MQC_E_OVERLAP) before any HIP call."""
    lib = nat.load()
    rows, dm, k, zs = 64, 72, 128, 144
    Y = 1 << 24
    W = Y + rows * k * 2 + 4096
    X = W + dm * k * 2 + 4096
    Z = X + rows * dm * 2 + 4096
    O = Z + rows * zs * 2 + 4096
    p = ctypes.c_void_p

    def call(out, bias=None):
        # (y, W, bias, x, z, z_row_stride, out, rows, d_model, k, dtype, stream)
        return lib.mqc_out_proj_gate_fwd(p(Y), p(W), p(bias) if bias else None, p(X), p(Z),
                                         zs, p(out), rows, dm, k, 1, None)

    for out in (Y + 16, W + 16, Z + (rows - 1) * zs * 2, X + 16, X - 16):
        assert call(out) == -7, hex(out)
    assert call(O, bias=O + rows * dm * 2 - 2) == -7


def test_fused_bc_split_workspace_without_gpu():
    """The split fused walk's workspace: two fp32 partial sums of y when there are
    two halves of states and steps to walk, none otherwise; a missing, short or
    misaligned workspace is refused before any HIP call."""
    lib = nat.load()
    assert lib.mqc_ssm_fused_bc_split_workspace_bytes(1, 2048, 1536, 64) == 2 * 2048 * 1536 * 16
    assert lib.mqc_ssm_fused_bc_split_workspace_bytes(3, 7, 64, 34) == 2 * 3 * 7 * 64 * 16
    assert lib.mqc_ssm_fused_bc_split_workspace_bytes(1, 2048, 1536, 32) == 0
    assert lib.mqc_ssm_fused_bc_split_workspace_bytes(1, 0, 1536, 64) == 0
    assert lib.mqc_ssm_fused_bc_split_workspace_bytes(-1, 2, 64, 64) == -2
    need = lib.mqc_ssm_fused_bc_split_workspace_bytes(1, 16, 64, 64)
    P = [FAKE] * 8 + [None, FAKE, None, 1, 16, 64, 64, 1e-6, 1]
    assert lib.mqc_ssm_fused_bc_fwd_split(*P, None, need, None) == -1
    assert lib.mqc_ssm_fused_bc_fwd_split(*P, FAKE, need - 1, None) == -6
    assert lib.mqc_ssm_fused_bc_fwd_split(*P, ctypes.c_void_p(4096 + 8), need, None) == -4


def test_fused_bc_validation_without_gpu():
    """mqc_ssm_fused_bc_fwd refuses, before any HIP call: fp32 or an unknown dtype
    (it runs bf16 and fp16), d_state odd or above 64, d_inner not a multiple of 64,
    NULL operands and misaligned pointers; nothing to do is not an error."""
    lib = nat.load()
    bf = 1
    odd = ctypes.c_void_p(4096 + 8)
    P = [FAKE] * 8  # x, W_B, W_C, delta, s, lambda_alpha, lambda_imag, D
    # (…, h0, y, h_last, batch, seq_len, d_inner, d_state, eps, dtype, stream)
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 1, 16, 64, 64, 1e-6, 0, None) == -3
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 1, 16, 64, 64, 1e-6, 3, None) == -3
    # fp16 passes the dtype check and stops at the next one (d_state odd).
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 1, 16, 64, 63, 1e-6, 2, None) == -2
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 1, 16, 64, 63, 1e-6, bf, None) == -2
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 1, 16, 64, 66, 1e-6, bf, None) == -5
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 1, 16, 96, 64, 1e-6, bf, None) == -2
    assert lib.mqc_ssm_fused_bc_fwd(None, *P[1:], None, FAKE, None, 1, 16, 64, 64, 1e-6, bf,
                                    None) == -1
    assert lib.mqc_ssm_fused_bc_fwd(odd, *P[1:], None, FAKE, None, 1, 16, 64, 64, 1e-6, bf,
                                    None) == -4
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, 0, 16, 64, 64, 1e-6, bf, None) == 0
    assert lib.mqc_ssm_fused_bc_fwd(*P, None, FAKE, None, -1, 16, 64, 64, 1e-6, bf, None) == -2


def test_auto_chunk_count_within_the_launch_limit():
    """The library's chunk length keeps batch * n_chunks within the chunked
    launches' 65535 rows, also for large batches of few states."""
    lib = nat.load()
    for b, T, d, k in ((8192, 4096, 4, 1), (4096, 2048, 1, 2), (65535, 512, 1, 1),
                       (1, 262144, 8, 64), (300, 100000, 1, 1)):
        L = lib.mqc_ssm_chunk_len_auto(b, T, d, k, 1)
        assert 1 <= L <= T
        assert b * -(-T // L) <= 65535 or L == T, (b, T, d, k, L)
        if L < T:
            assert lib.mqc_ssm_chunked_workspace_bytes(b, T, d, k, L) > 0


def test_gemm_validation_without_gpu():
    lib = nat.load()
    # bf16 or fp16; N a multiple of 256, K of 64; nothing to do is not an error.
    assert lib.mqc_gemm_nt(FAKE, FAKE, FAKE, 8, 256, 64, 0, None) == -3
    assert lib.mqc_gemm_nt(FAKE, FAKE, FAKE, 8, 200, 64, 2, None) == -2  # fp16 reaches the shape check
    assert lib.mqc_gemm_nt(FAKE, FAKE, FAKE, 8, 200, 64, 1, None) == -2
    assert lib.mqc_gemm_nt(FAKE, FAKE, FAKE, 8, 256, 96, 1, None) == -2
    assert lib.mqc_gemm_nt(None, FAKE, FAKE, 8, 256, 64, 1, None) == -1
    assert lib.mqc_gemm_nt(ctypes.c_void_p(4104), FAKE, FAKE, 8, 256, 64, 1, None) == -4
    assert lib.mqc_gemm_nt(None, None, None, 0, 256, 64, 1, None) == 0


def test_step_counter_limits_without_gpu():
    """The SSM kernels count steps in 32 bits and address D through a 32-bit
    lane offset: the entry points refuse T >= 2^30 and a negative D stride
    before any HIP call."""
    lib = nat.load()
    T = 1 << 30
    P = [FAKE] * 7
    assert lib.mqc_ssm_fused_fwd(*P, None, FAKE, None, 1, T, 2, 8, 1e-6, 1, None) == -5
    assert lib.mqc_ssm_q_fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, 1, None, FAKE, None,
                             1, T, 2, 8, 0, None) == -5
    assert lib.mqc_ssm_q_fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 0, -1, None, FAKE, None,
                             1, 4, 2, 8, 0, None) == -5
    assert lib.mqc_ssm_fused_fwd_train(*P, None, FAKE, None, FAKE, 8, 1, T, 2, 8,
                                       1e-6, 1, None) == -5
    G = [FAKE] * 7
    assert lib.mqc_ssm_fused_bwd(*P, None, FAKE, 8, FAKE, None, *G, None, 1, T, 2, 8,
                                 1e-6, 1, None) == -5


def test_empty_walk_validation_without_gpu():
    """seq_len 0 is work when the final state (or, in the backward, the
    parameter partials) must be written: the parameters are then required, the
    per-step operands are not; without an h_last buffer it is a no-op."""
    lib = nat.load()
    assert lib.mqc_ssm_fused_fwd(None, None, None, None, None, None, None, None, None, None,
                                 2, 0, 3, 8, 1e-6, 1, None) == 0
    assert lib.mqc_ssm_fused_fwd(None, None, None, None, None, None, None, None, None, FAKE,
                                 2, 0, 3, 8, 1e-6, 1, None) == -1
    assert lib.mqc_ssm_fused_fwd_train(None, None, None, None, None, None, None, None, None,
                                       FAKE, None, 8, 2, 0, 3, 8, 1e-6, 1, None) == -1
    assert lib.mqc_ssm_fused_bwd(None, None, None, None, None, None, None, None, None, 8, None,
                                 None, None, None, None, None, None, None, None, None,
                                 2, 0, 3, 8, 1e-6, 1, None) == -1


def test_block_seeded_init_matches_reference():
    info = json.loads((GOLDEN / "init_c1.json").read_text())
    torch.manual_seed(0)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    sd = blk.state_dict()
    assert sorted(sd) == sorted(info)
    for k, v in sd.items():
        a = v.detach().float().contiguous().numpy()
        assert list(a.shape) == info[k]["shape"], k
        assert hashlib.sha256(a.tobytes()).hexdigest() == info[k]["sha256"], k


def test_product_never_imports_oracle():
    pkg = ROOT / "mambaqc_amd"
    for f in pkg.rglob("*.py"):
        src = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", src, re.M), f
        assert "oracle." not in src.replace("# ", ""), f


def test_kernel_exports_are_functions():
    # `quaternion_norm` is both a submodule name and an exported function;
    # the export must be the function (reference kernels/__init__.py:10-33).
    import types
    for name in K.__all__:
        obj = getattr(K, name)
        assert not isinstance(obj, types.ModuleType), name
        assert callable(obj), name


def test_lm_seeded_init_matches_reference():
    """The LM re-draws every nn.Linear / nn.Embedding weight after the blocks'
    own initialisation, in module traversal order: same parameters, bit for bit,
    as the reference constructor under the same seed (tests/golden/init_lm.json)."""
    info = json.loads((GOLDEN / "init_lm.json").read_text())
    torch.manual_seed(0)
    lm = mambaqc_amd.QuaternionMamba2(37, d_model=16, n_layers=2, d_state=4, d_conv=4,
                                      expand_factor=2)
    sd = lm.state_dict()
    assert sorted(sd) == sorted(info)
    for k, v in sd.items():
        a = v.detach().float().contiguous().numpy()
        assert list(a.shape) == info[k]["shape"], k
        assert hashlib.sha256(a.tobytes()).hexdigest() == info[k]["sha256"], k
    assert lm.vocab_size_padded == 40
    assert lm.get_num_params() == sum(p.numel() for p in lm.parameters()) - 2 * 40 * 16


def test_lm_presets_shapes():
    # Constructed on the meta device: shapes only, no memory.
    with torch.device("meta"):
        base = mambaqc_amd.quaternion_mamba2_base(10000)
    n = sum(p.numel() for p in base.parameters())
    assert base.vocab_size_padded == 10000 and len(base.layers) == 12
    assert 14.6e9 < n < 14.7e9, n  # the B/C projections dominate


def test_param_f32_cache():
    """fp32 copies of parameters are reused while the parameter is unchanged,
    redone after an in-place update, skipped for fp32 parameters, and dropped
    with the parameter."""
    import gc
    p = torch.nn.Parameter(torch.randn(5, 3).bfloat16())
    a = nat.param_f32(p)
    assert a.dtype == torch.float32 and nat.param_f32(p) is a
    with torch.no_grad():
        p.add_(1)
    b = nat.param_f32(p)
    assert b is not a and torch.equal(b, p.detach().float())
    q = torch.nn.Parameter(torch.randn(4, 4))
    assert nat.param_f32(q).data_ptr() == q.data_ptr()
    key = id(p)
    assert key in nat._F32_CACHE
    del p, a, b
    gc.collect()
    assert key not in nat._F32_CACHE
    with torch.inference_mode():
        r = torch.randn(3, 2).bfloat16()
        assert torch.equal(nat.param_f32(r), r.float())


def test_build_rejects_kernels_that_spill():
    """The build reads the compiler's per-kernel resource remarks and refuses a
    kernel with scratch memory (a register spill): the parser finds the one
    kernel of a remark log that has scratch and none of those that have none."""
    from mambaqc_amd import build as B
    log = "\n".join([
        "In file included from x.hip:2:",
        "x.hpp:10:1: remark: Function Name: _Z4fastv [-Rpass-analysis=kernel-resource-usage]",
        "   10 | __global__ void fast() {",
        "      | ^",
        "x.hpp:10:1: remark:     VGPRs: 40 [-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:10:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:20:1: remark: Function Name: _Z4slowv [-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:20:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:20:1: remark:     ScratchSize [bytes/lane]: 116 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert B._spilling_kernels(log) == ["_Z4slowv (116 bytes/lane)"]
    assert B.RESOURCE_REMARKS == "-Rpass-analysis=kernel-resource-usage"


def test_wide_linear_block_rules():
    """Row blocks of the wide projections without a GPU: six 192 MiB blocks
    for a config-3 B/C weight in the forward, eight equal blocks for its
    batched input gradient (twelve for an fp32 weight), and no batched form
    when no count from the first candidate to four times it divides the rows."""
    from mambaqc_amd.layers import quaternion_linear as ql
    blocks = ql._blocks(393216, 1536, 2)
    assert len(blocks) == 6 and all(b - a == 65536 for a, b in blocks)
    assert ql._dx_batches(393216, 1536, 2) == 8
    assert ql._dx_batches(393216, 1536, 4) == 12
    assert ql._dx_batches(97, 1536, 2) == 0       # a prime row count
    assert ql._dx_batches(4 * 97, 1536, 2) == 0   # no count in 8..32 divides 388
    assert ql._dx_batches(8 * 97, 1536, 2) == 8


def test_bc_slice_rule():
    """The sliced B/C rule without a GPU: widths from the byte budget, whole
    projections below the bound, forced widths, and training slices refused
    beyond the backward's d_state limit."""
    import mambaqc_amd
    from mambaqc_amd import block as bm
    assert bm.bc_slice_width(1, 262144, 1536, 64, 2) == 8
    assert bm.bc_slice_width(4, 2048, 1536, 64, 2, budget=1) == 1
    assert bm.bc_slice_width(1, 4, 16, 4, 4, budget=1 << 40) == 16
    blk = mambaqc_amd.QuaternionMamba2Block(32, d_state=4)
    x = torch.zeros(2, 8, 64)
    with torch.no_grad():
        assert blk._bc_slice_width(x) == 0
        blk.bc_slice_d = 5
        assert blk._bc_slice_width(x) == 5
        blk.bc_slice_d = 1000
        assert blk._bc_slice_width(x) == 64
        blk.bc_slice_d = -1
        with pytest.raises(ValueError):
            blk._bc_slice_width(x)
    # Training slices too (the backward recomputes each slice's projections),
    # while d_state is within the backward's limit.
    blk.bc_slice_d = 5
    assert blk._bc_slice_width(x) == 5
    blk.bc_slice_d = None
    assert blk._bc_slice_width(x) == 0
    big = mambaqc_amd.QuaternionMamba2Block(16, d_state=128)
    big.bc_slice_d = 4
    with pytest.raises(ValueError, match="d_state <= 64"):
        big._bc_slice_width(torch.zeros(1, 4, 32))
    with torch.no_grad():
        assert big._bc_slice_width(torch.zeros(1, 4, 32)) == 4


def test_torch_ops_registered_with_fake_kernels():
    """Every kernel is a registered torch.ops.mambaqc op whose fake kernel gives
    the output shapes and dtypes on the meta device (no GPU, nothing runs);
    a CPU tensor reaching a real kernel raises instead of falling back."""
    from mambaqc_amd import ops

    mm = torch.ops.mambaqc
    for name in ops.OPS:
        assert hasattr(mm, name), name

    def m(*shape, dt=torch.float32):
        return torch.empty(*shape, device="meta", dtype=dt)

    bf = torch.bfloat16
    sh = lambda ts: [(tuple(t.shape), t.dtype) for t in (ts if isinstance(ts, (tuple, list)) else [ts])]
    assert sh(mm.quaternion_multiply(m(3, 5, 4), m(3, 5, 4))) == [((3, 5, 4), torch.float32)]
    assert sh(mm.quaternion_norm(m(3, 5, 4, dt=bf))) == [((3, 5), bf)]
    assert sh(mm.cumprod_scan(m(2, 7, 3, 2, 4))) == [((2, 7, 3, 2, 4), torch.float32)]
    assert sh(mm.ssm_forward_q(m(2, 7, 3, 2, 4), m(2, 7, 3, 2, 4), m(2, 7, 3, 4),
                               m(2, 7, 3, 2, 4), m(2, 7, 3))) == [((2, 7, 3, 4), torch.float32)]
    assert sh(mm.ssm_step_q(m(2, 3, 5, 4), m(2, 3, 5, 4), m(2, 3, 4), m(2, 3, 5, 4), m(2, 3),
                            m(2, 3, 5, 4))) == [((2, 3, 5, 4), torch.float32), ((2, 3, 4), torch.float32)]
    dl = (m(2, 17, 3, dt=bf), m(2, 17, 3, dt=bf), m(2, 17, 3, 4, 4, dt=bf), m(2, 17, 3, 4, 4, dt=bf),
          m(3, 4), m(3, 4, 3), m(3))
    assert sh(mm.ssm_forward_dl(*dl)) == [((2, 17, 3, 4), bf), ((2, 3, 4, 4), torch.float32)]
    # 16-bit storage: a checkpoint every 8 steps.
    assert sh(mm.ssm_forward_dl_train(*dl)) == [((2, 17, 3, 4), bf), ((2, 3, 4, 4), torch.float32),
                                                ((2, 3, 3, 4, 4), torch.float32)]
    g = mm.ssm_backward_dl(*dl, None, m(2, 3, 3, 4, 4), m(2, 17, 3, 4, dt=bf), None)
    assert sh(g) == [((2, 17, 3), torch.float32)] * 2 + [((2, 17, 3, 4, 4), bf)] * 2 + [
        ((3, 4), torch.float32), ((3, 4, 3), torch.float32), ((3,), torch.float32),
        ((0,), torch.float32)]
    assert sh(mm.ssm_front(m(2, 5, 3, dt=bf), m(2, 5, 3, dt=bf), m(2, 5, 3))) == [((2, 5, 3), torch.float32)] * 2
    assert sh(mm.quaternion_layer_norm(m(2, 5, 3, 4, dt=bf), m(3), m(3, 4))) == [
        ((2, 5, 3, 4), bf), ((2, 5), torch.float32), ((2, 5), torch.float32)]
    assert sh(mm.causal_conv1d_silu(m(2, 5, 3, dt=bf), m(3, 1, 4), m(3))) == [((2, 5, 3), bf)]
    assert sh(mm.causal_conv1d_silu_backward(m(2, 5, 3, dt=bf), m(3, 1, 4), None, m(2, 5, 3, dt=bf))) == [
        ((2, 5, 3), bf), ((3, 4), torch.float32), ((3,), torch.float32)]
    assert sh(mm.out_gate(m(2, 5, 8), m(2, 5, 16, dt=bf), m(2, 5, 8, dt=bf))) == [((2, 5, 8), torch.float32)]
    with pytest.raises(RuntimeError):
        mm.quaternion_multiply(torch.zeros(2, 4), torch.zeros(2, 4))


def test_param_f32_cache_under_inference_mode():
    """fp32 copies of 16-bit parameters are cached also when the call comes
    from inference mode (made as ordinary tensors), and redone after an
    in-place update; tensors made in inference mode convert every time."""
    p = torch.nn.Parameter(torch.randn(8, 3).to(torch.bfloat16))
    with torch.inference_mode():
        a = nat.param_f32(p)
        b = nat.param_f32(p)
    assert a is b and not a.is_inference() and a.dtype == torch.float32
    assert torch.equal(a, p.detach().float())
    with torch.no_grad():
        p.add_(1)
    c = nat.param_f32(p)
    assert c is not a and torch.equal(c, p.detach().float())
    with torch.inference_mode():
        t = torch.randn(4).to(torch.bfloat16)
        assert nat.param_f32(t) is not nat.param_f32(t)


def test_skinny_gemm_validation_without_gpu():
    """mqc_gemm_skinny_nt refuses bad sizes, dtypes, NULLs and misaligned
    pointers before any HIP call."""
    lib = nat.load()
    bf = 1
    odd = ctypes.c_void_p(4096 + 8)
    # (X, M, K, W1, bias1, Y1, N1, W2, bias2, Y2, N2, dtype, stream)
    assert lib.mqc_gemm_skinny_nt(FAKE, 17, 64, FAKE, None, FAKE, 8, None, None, None, 0, bf, None) == -5
    assert lib.mqc_gemm_skinny_nt(FAKE, 4, 48, FAKE, None, FAKE, 8, None, None, None, 0, bf, None) == -5
    assert lib.mqc_gemm_skinny_nt(FAKE, 4, 0, FAKE, None, FAKE, 8, None, None, None, 0, bf, None) == -5
    assert lib.mqc_gemm_skinny_nt(FAKE, 16, 4096, FAKE, None, FAKE, 8, None, None, None, 0, bf, None) == -5
    assert lib.mqc_gemm_skinny_nt(FAKE, 4, 64, FAKE, None, FAKE, 8, None, None, None, 0, 0, None) == -3
    assert lib.mqc_gemm_skinny_nt(FAKE, 4, 64, None, None, FAKE, 8, None, None, None, 0, bf, None) == -1
    assert lib.mqc_gemm_skinny_nt(FAKE, 4, 64, FAKE, None, FAKE, 8, FAKE, None, None, 8, bf, None) == -1
    assert lib.mqc_gemm_skinny_nt(odd, 4, 64, FAKE, None, FAKE, 8, None, None, None, 0, bf, None) == -4
    assert lib.mqc_gemm_skinny_nt(FAKE, -1, 64, FAKE, None, FAKE, 8, None, None, None, 0, bf, None) == -2
    assert lib.mqc_gemm_skinny_nt(None, 0, 64, None, None, None, 8, None, None, None, 0, bf, None) == 0


def test_conv_step_validation_without_gpu():
    """mqc_causal_conv_silu_step refuses bad sizes, NULLs and misaligned
    pointers before any HIP call."""
    lib = nat.load()
    bf = 1
    odd = ctypes.c_void_p(4096 + 1)
    # (x, x_row_stride, tail, w, bias, out, batch, channels, kernel, dtype, stream)
    assert lib.mqc_causal_conv_silu_step(FAKE, 16, FAKE, FAKE, None, FAKE, 2, 16, 0, bf, None) == -2
    assert lib.mqc_causal_conv_silu_step(FAKE, 8, FAKE, FAKE, None, FAKE, 2, 16, 4, bf, None) == -2
    assert lib.mqc_causal_conv_silu_step(FAKE, 16, FAKE, FAKE, None, FAKE, 2, 16, 9, bf, None) == -5
    assert lib.mqc_causal_conv_silu_step(FAKE, 16, None, FAKE, None, FAKE, 2, 16, 4, bf, None) == -1
    assert lib.mqc_causal_conv_silu_step(FAKE, 16, FAKE, FAKE, None, FAKE, 2, 16, 4, 7, None) == -3
    assert lib.mqc_causal_conv_silu_step(odd, 16, FAKE, FAKE, None, FAKE, 2, 16, 4, bf, None) == -4
    assert lib.mqc_causal_conv_silu_step(None, 16, None, None, None, None, 0, 16, 4, bf, None) == 0


def test_chunked_walks_check_before_any_launch():
    """The chunked entry points run the walk's own argument checks (alignment,
    32-bit slice offsets) before their first launch: without a GPU they return
    the check's code, not a HIP error from a carry launch that ran first."""
    lib = nat.load()
    bf = 1
    K = lib.mqc_ssm_bwd_ckpt_every(bf)
    odd = ctypes.c_void_p(4096 + 2)  # 2-byte aligned: too little for 8-byte B loads
    big = 1 << 40
    # Inference: (delta, s, B, C, la, li, D, h0, y, h_last, batch, T, d, S, L, eps, dtype, ws, bytes, stream)
    # (h0 NULL: a chunked walk refuses h_last over h0.)
    P = [FAKE, FAKE, odd] + [FAKE] * 4 + [None, FAKE, FAKE]
    assert lib.mqc_ssm_fused_fwd_chunked(*P, 1, 200, 8, 64, 64, 1e-6, bf, FAKE, big, None) == -4
    P = [FAKE] * 7 + [None, FAKE, FAKE]
    # 2^22 d's x 64 states x 4 x 2 bytes = 2 GiB per (b, t) slice: past the 32-bit offsets.
    assert lib.mqc_ssm_fused_fwd_chunked(*P, 1, 200, 1 << 22, 64, 64, 1e-6, bf, FAKE, big, None) == -5
    # Training forward: 11 pointers (… h_last, h_ckpt), then ckpt_every.
    P = [FAKE, FAKE, odd] + [FAKE] * 4 + [None] + [FAKE] * 3
    assert lib.mqc_ssm_fused_fwd_train_chunked(*P, K, 1, 200, 8, 64, 64, 1e-6, bf, FAKE, big, None) == -4
    # Backward: 9 pointers, ckpt_every, 10 pointers (gy first).
    Q = [FAKE] * 9
    R = [odd] + [FAKE] * 8 + [None]  # dh0 NULL (it may not overlap dh_last)
    assert lib.mqc_ssm_fused_bwd_chunked(*Q, K, *R, 1, 200, 8, 64, 64, 1e-6, bf, FAKE, big, None) == -4
    R = [FAKE] * 9 + [None]
    assert lib.mqc_ssm_fused_bwd_chunked(*Q, K, *R, 1, 200, 1 << 22, 64, 64, 1e-6, bf, FAKE, big,
                                         None) == -5


def test_chunked_training_validation_without_gpu():
    """The chunked training entry points refuse, before any HIP call, a chunk
    length that is not a multiple of the checkpoint interval, a short
    workspace and d_state above 64; the Python rule rounds chunk lengths up to
    that interval."""
    from mambaqc_amd.kernels.ssm_fused import train_chunk_len
    lib = nat.load()
    bf = 1
    K = lib.mqc_ssm_bwd_ckpt_every(bf)
    assert K == 8
    P = [FAKE] * 11
    # (…, ckpt_every, batch, seq_len, d_inner, d_state, chunk_len, eps, dtype, ws, ws_bytes, stream)
    assert lib.mqc_ssm_fused_fwd_train_chunked(*P, K, 1, 100, 4, 8, 12, 1e-6, bf, FAKE, 1 << 20, None) == -2
    assert lib.mqc_ssm_fused_fwd_train_chunked(*P, K, 1, 100, 4, 8, 0, 1e-6, bf, FAKE, 1 << 20, None) == -2
    assert lib.mqc_ssm_fused_fwd_train_chunked(*P, K, 1, 100, 4, 8, 16, 1e-6, bf, FAKE, 0, None) == -6
    assert lib.mqc_ssm_fused_fwd_train_chunked(*P, K, 1, 100, 4, 128, 16, 1e-6, bf, FAKE, 1 << 30, None) == -5
    Q = [FAKE] * 9
    R = [FAKE] * 10
    assert lib.mqc_ssm_fused_bwd_chunked(*Q, K, *R, 1, 100, 4, 8, 12, 1e-6, bf, FAKE, 1 << 20, None) == -2
    assert lib.mqc_ssm_fused_bwd_chunked(*Q, K, *R, 1, 100, 4, 8, 16, 1e-6, bf, FAKE, 16, None) == -6
    assert lib.mqc_ssm_fused_bwd_chunked(*Q, K, *R, 1, 100, 4, 8, 16, 1e-6, bf, None, 1 << 30, None) == -1
    assert train_chunk_len(1, 2048, 1536, 64, torch.bfloat16) % 8 == 0
    assert train_chunk_len(1, 2048, 1536, 64, torch.float32) % 4 == 0
    assert train_chunk_len(1, 100, 4, 8, torch.bfloat16, chunk_len=13) == 16
    assert train_chunk_len(4, 2048, 1536, 64, torch.bfloat16) >= 2048  # config 3: whole
