"""GPU parity of the hand-written MFMA GEMM (mqc_gemm_nt, bf16 and fp16): ragged M
(rows past M are clamped for the loads and never stored), several N and K, against
float64 torch on the same 16-bit inputs; and the config-3 B/C projection shape
against torch's own GEMM."""
import pytest
import torch

from conftest import assert_close

from mambaqc_amd import _native as nat

pytestmark = pytest.mark.gpu
DEV = "cuda"


def gemm(X, W):
    M, K = X.shape
    N = W.shape[0]
    C = torch.full((M, N), float("nan"), device=DEV, dtype=X.dtype)
    nat.call("mqc_gemm_nt", X, X.data_ptr(), W.data_ptr(), C.data_ptr(), M, N, K,
             nat.dtype_code(X), nat.stream_of(X))
    return C


@pytest.mark.parametrize("M,N,K", [(1, 256, 64), (5, 512, 128), (255, 256, 192), (257, 768, 1536),
                                   (1000, 1024, 320), (2048, 8192, 1536), (300, 256, 64)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_gemm_vs_fp64(M, N, K, dt):
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    X = torch.randn(M, K, generator=g, device=DEV).to(dt)
    W = (torch.randn(N, K, generator=g, device=DEV) * 0.05).to(dt)
    C = gemm(X, W)
    assert C.dtype == dt
    ref = X.double() @ W.double().t()
    # One 16-bit rounding of an fp32 accumulation: rtol 1e-2 with the atol floor.
    assert_close(C, ref, 1e-2, f"gemm {M}x{N}x{K} {dt}")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_gemm_config3_projection_shape(dt):
    """M 8192 (B4 x T2048), N 393216 (d_inner 1536 x d_state 64 x 4), K 1536:
    against torch's GEMM (hipBLASLt) on the same inputs, and row 4321 against
    float64."""
    g = torch.Generator(device=DEV).manual_seed(0)
    X = torch.randn(8192, 1536, generator=g, device=DEV).to(dt)
    W = (torch.randn(393216, 1536, generator=g, device=DEV) * 0.02).to(dt)
    C = gemm(X, W)
    ref = torch.mm(X, W.t())
    err = (C.float() - ref.float()).abs().max().item()
    scale = ref.float().abs().max().item()
    assert err <= 1e-2 * scale, (err, scale)
    row = (X[4321].double() @ W.double().t()).view(1, -1)
    assert_close(C[4321:4322], row, 1e-2, "row 4321 vs fp64")
