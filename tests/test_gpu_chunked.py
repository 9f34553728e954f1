"""GPU parity of the time-chunked SSM walk (mqc_ssm_fused_fwd_chunked): the T
axis cut into chunks that are reduced to transitions (P, H), combined by a
wave-level associative scan, and walked from their start states. Checked
against the CPU oracle's sequential walk and against the whole walk on the
same device, over chunk counts that hit every scan segment width (1 to 64
lanes and two rounds of 64), ragged last chunks, chunk length 1, and an
order known-answer test routed through the carry scan.
"""
import pytest
import torch

import oracle
from conftest import assert_close, tol

from mambaqc_amd import kernels as K
from mambaqc_amd.kernels.ssm_fused import chunk_len_for

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _dl_inputs(b, T, d, k, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    delta = torch.nn.functional.softplus(r(b, T, d) - 2).to(dtype)
    s = r(b, T, d).to(dtype)
    Bm = (r(b, T, d, k, 4) * 0.1).to(dtype)
    C = (r(b, T, d, k, 4) * 0.1).to(dtype)
    la = r(d, k) * 0.5 + 1
    li = r(d, k, 3) * 0.1
    D = torch.ones(d) + 0.1 * r(d)
    h0 = r(b, d, k, 4) * 0.3
    return (delta, s, Bm, C, la, li, D), h0


def up(t):
    return t.detach().cpu().double()


# (shape (b, T, d_inner, d_state), chunk_len): carries nc = ceil(T / L) - 1 set
# the scan's segment width (smallest power of two >= nc, at most 64).
CASES = [
    ((1, 33, 9, 64), 32),      # 2 chunks, the last of one step: segment 1
    ((3, 41, 2, 1), 20),       # d_state 1, last chunk of one step: segment 2
    ((1, 64, 8, 64), 16),      # 4 chunks: segment 4
    ((2, 37, 5, 16), 10),      # ragged last chunk (7 steps): segment 4
    ((1, 50, 13, 32), 7),      # 8 chunks, last of one step: segment 8
    ((1, 170, 5, 16), 10),     # 17 chunks: segment 16
    ((2, 100, 3, 8), 4),       # 25 chunks: segment 32 (row_bcast:15)
    ((1, 300, 4, 64), 9),      # 34 chunks: segment 64 (row_bcast:15 and :31)
    ((1, 70, 3, 4), 1),        # chunk length 1: 69 carries, two rounds of 64
    ((2, 200, 6, 64), 2),      # 99 carries, two rounds
    ((8, 130, 768, 64), 33),   # enough states for several per lane in both walks
]


@pytest.mark.parametrize("shape,L", CASES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_chunked_vs_oracle(shape, L, dtype):
    ins, h0 = _dl_inputs(*shape, seed=sum(shape) + L, dtype=dtype)
    dev = [t.to(DEV) for t in ins]
    y, h = K.ssm_forward_fused_dl(*dev, h0=h0.to(DEV), return_state=True, chunk_len=L)
    ry, rh = oracle.ssm_forward_dl_reference(*(up(t) for t in ins), h0=up(h0), return_state=True)
    assert_close(y, ry, tol(dtype), f"chunked y {shape} L={L} {dtype}")
    assert_close(h, rh, tol(dtype), f"chunked h_last {shape} L={L} {dtype}")
    # Against the whole walk on the device: the same arithmetic in another
    # order, so they agree to rounding.
    yw, hw = K.ssm_forward_fused_dl(*dev, h0=h0.to(DEV), return_state=True, chunk_len=shape[1])
    assert_close(y, yw, tol(dtype), f"chunked vs whole y {shape} L={L} {dtype}")
    assert_close(h, hw, 1e-4, f"chunked vs whole h {shape} L={L} {dtype}")


def _order_case(T):
    """d_state 1, Lambda along i, B = j at t = 0 and 0 after, C = 1, D = 0,
    s = 1: the state is h_t = (q_t ... q_1) (x) j, and y_t = h_t."""
    delta = (0.2 + 0.05 * torch.arange(T, dtype=torch.float32)).view(1, T, 1)
    s = torch.ones(1, T, 1)
    Bm = torch.zeros(1, T, 1, 1, 4)
    Bm[0, 0, 0, 0, 2] = 1.0
    C = torch.zeros(1, T, 1, 1, 4)
    C[..., 0] = 1.0
    la = torch.tensor([[0.3]])
    li = torch.tensor([[[0.7, 0.0, 0.0]]])
    D = torch.zeros(1)
    return delta, s, Bm, C, la, li, D


@pytest.mark.parametrize("T,L", [(3, 1), (70, 1), (40, 3)])
def test_ssm_chunked_order_kat(T, L):
    """The carry scan composes the later transition on the left. With q_t in
    the plane of i and a state along j, q (x) j = q_w j + q_x k while
    j (x) q = q_w j - q_x k: the sign of the k component tells the order.
    Expected y_t = cumprod(q)_t (x) j, with the cumulative product from the
    oracle's cumprod (pinned by its own known answers) and (x) j from the
    multiplication table: (w + x i)(j) = (0, 0, w, x)."""
    ins = _order_case(T)
    y = K.ssm_forward_fused_dl(*(t.to(DEV) for t in ins), chunk_len=L)
    lam = oracle.lambda_from_params(ins[4].double(), ins[5].double())  # [1, 1, 4]
    z = ins[0].double().view(1, T, 1, 1) * lam.view(1, 1, 1, 4)        # [1, T, 1, 4]
    q = oracle.cayley_reference(z)
    # h_0 = s_0 B_0 = j (q_0 acts on the zero state), then h_t = q_t (x) h_{t-1}:
    # the product runs over q_1 .. q_t.
    cum1 = oracle.cumprod_reference(q[:, 1:]).view(T - 1, 4)
    want = torch.zeros(T, 4, dtype=torch.float64)
    want[0] = torch.tensor([0.0, 0.0, 1.0, 0.0])
    want[1:, 2] = cum1[:, 0]
    want[1:, 3] = cum1[:, 1]
    assert (cum1[:, 2:].abs() < 1e-12).all()  # products stay in the plane of i
    got = y.view(T, 4).double().cpu()
    assert_close(got, want, 1e-5, f"order KAT T={T} L={L}")
    # The reversed composition would flip the k component.
    assert (got[1:, 3] * cum1[:, 1] > 0).all()


def test_ssm_chunked_auto_path_matches_whole_walk():
    """With the library's choice (chunk_len=None) a batch-1 walk is chunked and
    agrees with the whole walk."""
    shape = (1, 512, 96, 64)
    ins, h0 = _dl_inputs(*shape, seed=5, dtype=torch.bfloat16)
    dev = [t.to(DEV) for t in ins]
    assert chunk_len_for(1, 512, 96, 64, torch.bfloat16) < 512
    y = K.ssm_forward_fused_dl(*dev)
    yw = K.ssm_forward_fused_dl(*dev, chunk_len=512)
    assert_close(y, yw, 2e-2, "auto chunked vs whole")
