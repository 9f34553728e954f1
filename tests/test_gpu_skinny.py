"""GPU tests of the skinny GEMM of decode-sized products (mqc_gemm_skinny_nt):
against float64 on ragged shapes, with and without bias, single and paired
weights, 1 to 16 rows, in bf16 and fp16; the eligibility rule's fallbacks; and
the block's projections on it against F.linear."""
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_close
from mambaqc_amd import _native as nat
from mambaqc_amd.layers import quaternion_linear as ql

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
# Few tiles and long K take the split modes (waves sharing a tile's K):
# (4, 768, 200) 4 waves, (4, 1536, 1000) and (4, 6144, 768) 8 (the latter held
# there by LDS), (2, 4096, 40) 16; many tiles, or short K, one wave per tile.
# At least 4096 groups of 8 weight rows, at most 8 token rows and K a multiple
# of 64 take the wide mode: unrolled lines (K 1024, 1536, 2048) with 1, 2, 4
# and 8 padded token rows, lines in groups of 8 (K 640, 4096), ragged N, the
# 4096-group boundary; (12, 1536, 40000) has too many rows and stays in tiles.
@pytest.mark.parametrize("M,K,N1,N2,bias", [(1, 64, 48, 0, False), (4, 1536, 1000, 0, True),
                                            (16, 96, 33, 17, True), (3, 1536, 4096, 4096, False),
                                            (7, 2016, 77, 5, True), (4, 256, 16, 16, False),
                                            (2, 32, 1, 0, True), (4, 768, 200, 0, True),
                                            (2, 4096, 40, 24, False), (4, 6144, 768, 0, True),
                                            (4, 1024, 40000, 40000, False),
                                            (4, 1536, 40000, 40003, False), (1, 1024, 33001, 0, True),
                                            (8, 2048, 20000, 20001, True), (5, 640, 40007, 0, True),
                                            (3, 4096, 33000, 0, False), (2, 1536, 16384, 16384, True),
                                            (12, 1536, 40000, 0, False)])
def test_skinny_vs_float64(dtype, M, K, N1, N2, bias):
    g = torch.Generator(device=DEV).manual_seed(M * 1000 + K + N1)
    x = torch.randn(M, K, generator=g, device=DEV).to(dtype)
    w1 = (torch.randn(N1, K, generator=g, device=DEV) * 0.05).to(dtype)
    b1 = (torch.randn(N1, generator=g, device=DEV) * 0.1).to(dtype) if bias else None
    w2 = (torch.randn(N2, K, generator=g, device=DEV) * 0.05).to(dtype) if N2 else None
    b2 = (torch.randn(N2, generator=g, device=DEV) * 0.1).to(dtype) if (bias and N2) else None
    assert ql.skinny_eligible(x, w1, b1, *(() if w2 is None else (w2, b2)))
    out = ql.skinny_linear(x, w1, b1, w2, b2)
    y1, y2 = out if w2 is not None else (out, None)
    ref = lambda w, b: x.double() @ w.double().t() + (0 if b is None else b.double())
    assert_close(y1, ref(w1, b1), 1e-2, f"y1 {dtype} M{M} K{K} N{N1}")
    if w2 is not None:
        assert_close(y2, ref(w2, b2), 1e-2, f"y2 {dtype} M{M} K{K} N{N2}")


def test_skinny_eligibility():
    x = torch.randn(4, 64, device=DEV).bfloat16()
    w = torch.randn(32, 64, device=DEV).bfloat16()
    assert ql.skinny_eligible(x, w, None)
    assert not ql.skinny_eligible(x.float(), w.float(), None)            # fp32
    assert not ql.skinny_eligible(torch.randn(17, 64, device=DEV).bfloat16(), w, None)  # rows
    assert not ql.skinny_eligible(x[:, :48], w[:, :48].contiguous(), None)  # K % 32
    assert not ql.skinny_eligible(x, w.t().contiguous().t(), None)       # strided weight
    assert not ql.skinny_eligible(x, w.requires_grad_(), None)           # autograd
    with torch.no_grad():
        assert ql.skinny_eligible(x, w, None)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert not ql.skinny_eligible(x, w.detach(), None)
    # Weights past the bound stay off the skinny GEMM unless its wide mode
    # applies (at most 8 rows, K a multiple of 64).
    big = torch.empty(ql.SKINNY_MAX_WEIGHT_BYTES // 192 + 1, 96, device=DEV, dtype=torch.bfloat16)
    assert not ql.skinny_eligible(torch.randn(4, 96, device=DEV).bfloat16(), big, None)  # K % 64
    del big
    big = torch.empty(ql.SKINNY_MAX_WEIGHT_BYTES // 128 + 1, 64, device=DEV, dtype=torch.bfloat16)
    assert ql.skinny_eligible(x, big, None)
    assert not ql.skinny_eligible(torch.randn(9, 64, device=DEV).bfloat16(), big, None)  # rows


def test_skinny_entry_point_limits():
    """K not a multiple of 32 and more than 16 rows are refused by the entry point itself."""
    x = torch.randn(4, 48, device=DEV).bfloat16()
    w = torch.randn(8, 48, device=DEV).bfloat16()
    y = torch.empty(4, 8, device=DEV).bfloat16()
    lib = nat.load()
    assert lib.mqc_gemm_skinny_nt(x.data_ptr(), 4, 48, w.data_ptr(), None, y.data_ptr(), 8, None,
                                  None, None, 0, 1, None) == -5
    x = torch.randn(17, 64, device=DEV).bfloat16()
    w = torch.randn(8, 64, device=DEV).bfloat16()
    y = torch.empty(17, 8, device=DEV).bfloat16()
    assert lib.mqc_gemm_skinny_nt(x.data_ptr(), 17, 64, w.data_ptr(), None, y.data_ptr(), 8, None,
                                  None, None, 0, 1, None) == -5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_block_decode_projections_on_skinny(dtype):
    """A block at decode size (4 token rows, no autograd) computes its
    projections on the skinny GEMM; its output agrees with F.linear-based
    projections to the operands' rounding."""
    import mambaqc_amd
    from mambaqc_amd import block as bm
    torch.manual_seed(3)
    with torch.device(DEV):
        blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    blk = blk.to(dtype).eval()
    x = torch.randn(4, 1, 64, device=DEV).to(dtype)
    calls = []
    real = ql.skinny_linear
    try:
        bm.skinny_linear = lambda *a, **k: calls.append(1) or real(*a, **k)
        with torch.no_grad():
            got = blk(x)
    finally:
        bm.skinny_linear = real
    assert len(calls) == 4  # in_proj, dt/gate pair, B/C pair, out_proj
    eligible = ql.skinny_eligible
    try:
        bm.skinny_eligible = lambda *a, **k: False
        with torch.no_grad():
            want = blk(x)
    finally:
        bm.skinny_eligible = eligible
    assert_close(got, want, 2e-2, f"block decode projections {dtype}")
