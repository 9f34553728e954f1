"""GPU parity: every HIP kernel of libmambaqc_hip.so against the CPU oracle on
identical seeded inputs. fp32 within rtol 1e-4, bf16/fp16 within 2e-2 (both
with an atol floor of rtol * max|ref|); 16-bit cases compare against the
oracle run in fp32/fp64 on the same rounded inputs.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN, assert_close, tol

import mambaqc_amd
from mambaqc_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def rnd(*shape, seed=0, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def up(t):
    return t.detach().cpu().double()


def test_native_library_is_the_compute_path():
    p = rnd(64, 4).to(DEV)
    K.quaternion_multiply(p, p)
    torch.cuda.synchronize()
    maps = open("/proc/self/maps").read()
    assert "libmambaqc_hip.so" in maps


# ---------------------------------------------------------------- element-wise
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [0, 1, 37, 4096 + 3])
def test_quaternion_multiply(dtype, n):
    p, q = rnd(n, 4, seed=1, dtype=dtype), rnd(n, 4, seed=2, dtype=dtype)
    got = K.quaternion_multiply(p.to(DEV), q.to(DEV))
    assert got.dtype == dtype and got.shape == p.shape
    assert_close(got, oracle.hamilton(up(p), up(q)), tol(dtype), f"qmul {dtype} n={n}")


def test_quaternion_multiply_table_exact():
    e = torch.eye(4, device=DEV)
    p = e.repeat_interleave(4, 0)
    q = e.repeat(4, 1)
    got = K.quaternion_multiply(p, q).cpu()
    want = oracle.hamilton(p.cpu(), q.cpu())
    assert torch.equal(got, want)


def test_quaternion_multiply_batched_and_views():
    p = rnd(2, 3, 5, 7, 4, seed=3)
    q = rnd(2, 3, 5, 7, 4, seed=4)
    got = K.quaternion_multiply_batched(p.to(DEV), q.to(DEV))
    assert_close(got, oracle.hamilton(up(p), up(q)), 1e-4, "qmul batched")
    # Non-contiguous and misaligned views are accepted.
    big = rnd(9, 4, seed=5).to(DEV)
    got = K.quaternion_multiply(big[1:8], big[2:9])
    assert_close(got, oracle.hamilton(up(big[1:8]), up(big[2:9])), 1e-4, "qmul offset views")


@pytest.mark.parametrize("dtype", DTYPES)
def test_conjugate_inverse_norm(dtype):
    q = rnd(3, 11, 4, seed=6, dtype=dtype)
    qd = q.to(DEV)
    assert_close(K.quaternion_conjugate(qd), oracle.conjugate(up(q)), tol(dtype), "conj")
    assert_close(K.quaternion_inverse(qd), oracle.inverse(up(q)), tol(dtype), "inv")
    assert_close(K.quaternion_norm(qd), oracle.norm(up(q)), tol(dtype), "norm")
    tiny = torch.tensor([[1e-4, 0.0, 0.0, 0.0]], device=DEV)
    assert_close(K.quaternion_inverse(tiny, eps=1e-6), oracle.inverse(tiny.cpu(), 1e-6), 1e-4, "inv clamp")


# ---------------------------------------------------------------- Cayley
def test_cayley_golden():
    d = np.load(GOLDEN / "cayley.npz")
    z = torch.from_numpy(d["z"])
    got = K.cayley_discretization_fused(z.to(DEV), eps=float(d["eps"]))
    assert_close(got, torch.from_numpy(d["q"]), 1e-4, "cayley golden")


@pytest.mark.parametrize("dtype", DTYPES)
def test_cayley_random(dtype):
    z = rnd(2, 8, 16, 32, 4, seed=7, dtype=dtype)
    z[..., 0] = -z[..., 0].abs()
    got = K.cayley_discretization_fused(z.to(DEV))
    assert_close(got, oracle.cayley_reference(up(z)), tol(dtype), f"cayley {dtype}")


def test_cayley_identity_and_stability():
    z = torch.zeros(2, 4, 8, 16, 4, device=DEV)
    q = K.cayley_discretization_fused(z)
    want = torch.zeros_like(q)
    want[..., 0] = 1
    assert torch.equal(q, want)
    z = rnd(2, 4, 8, 16, 4, seed=8).to(DEV)
    z[..., 0] = -z[..., 0].abs() - 0.5
    assert (K.quaternion_norm(K.cayley_discretization_fused(z)) < 1.0 + 1e-4).all()


# ---------------------------------------------------------------- cumulative product
@pytest.mark.parametrize("shape", [(2, 37, 5, 7), (1, 300, 3, 64), (3, 1, 2, 3), (1, 64, 1, 1), (1, 129, 130, 1)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_cumprod(shape, dtype):
    b, T, d, k = shape
    # Unit-norm-ish factors keep the product's magnitude O(1) over long T.
    q = rnd(b, T, d, k, 4, seed=sum(shape), dtype=torch.float64)
    q = (q / q.norm(dim=-1, keepdim=True)).to(dtype)
    got = K.parallel_scan_quaternion(q.to(DEV))
    assert got.dtype == dtype
    assert_close(got, oracle.cumprod_reference(up(q)), tol(dtype), f"cumprod {shape} {dtype}")


def test_cumprod_order_and_identity():
    i = torch.tensor([0.0, 1, 0, 0])
    j = torch.tensor([0.0, 0, 1, 0])
    q = torch.stack([i, j]).view(1, 2, 1, 1, 4).to(DEV)
    out = K.parallel_scan_quaternion(q).cpu().view(2, 4)
    assert torch.equal(out[1], torch.tensor([0.0, 0, 0, -1]))
    ident = torch.zeros(2, 10, 8, 16, 4, device=DEV)
    ident[..., 0] = 1
    assert torch.equal(K.parallel_scan_quaternion(ident), ident)
    empty = torch.zeros(2, 0, 3, 4, 4, device=DEV)
    assert K.parallel_scan_quaternion(empty).shape == empty.shape


def test_cumprod_config2_full_size():
    """[2,256,768,64,4] fp32 (config 2): q = Cayley(z), then the scan. A lane
    slice is checked against the oracle; every lane is checked through
    |cum_t| = prod_{u<=t} |q_u| (norm multiplicativity)."""
    g = torch.Generator(device=DEV).manual_seed(0)
    shape = (2, 256, 768, 64)
    n = lambda: torch.randn(*shape, generator=g, device=DEV)
    z = torch.empty(*shape, 4, device=DEV)
    z[..., 0] = -torch.exp(n()) * torch.nn.functional.softplus(n())
    for c in range(1, 4):
        z[..., c] = n() * torch.nn.functional.softplus(n())
    q = K.cayley_discretization_fused(z)
    cum = K.parallel_scan_quaternion(q)
    sl = (slice(None), slice(None), slice(100, 103), slice(None))
    assert_close(q[sl], oracle.cayley_reference(z[sl].cpu()), 1e-4, "C2 cayley slice")
    assert_close(cum[sl], oracle.cumprod_reference(q[sl].cpu()), 1e-4, "C2 scan slice")
    # |q| < 1 at every step (Re z < 0), so the products decay and fall below
    # fp32's normal range (e^-87) after ~100 steps for about half the lanes.
    # Norms are taken in float64 (squares of fp32 values near 1e-20 would
    # underflow in fp32); multiplicativity is checked where the exact product
    # is a normal fp32 with margin, and decay is checked everywhere else.
    logn = torch.log(q.double().norm(dim=-1)).cumsum(1)
    got = torch.log(cum.double().norm(dim=-1))
    live = logn > -80.0
    assert live.float().mean().item() > 0.3, "too few lanes left to check"
    err = (got[live] - logn[live]).abs().max().item()
    assert err < 1e-3, f"norm multiplicativity violated: max |log| error {err}"
    dead = logn < -95.0
    assert (got[dead] < -85.0).all(), "products that must have decayed did not"


# ---------------------------------------------------------------- SSM (materialised q)
def _q_inputs(b, T, d, k, seed, dtype):
    q = rnd(b, T, d, k, 4, seed=seed, dtype=torch.float64)
    q = 0.9 * q / q.norm(dim=-1, keepdim=True)          # stable: |q| < 1
    Bm = rnd(b, T, d, k, 4, seed=seed + 1, scale=0.5, dtype=torch.float64)
    C = rnd(b, T, d, k, 4, seed=seed + 2, scale=0.5, dtype=torch.float64)
    S = rnd(b, T, d, 4, seed=seed + 3, dtype=torch.float64)
    D = rnd(d, seed=seed + 4, dtype=torch.float64)
    return [t.to(dtype) for t in (q, Bm, S, C)] + [D.to(dtype)]


@pytest.mark.parametrize("k", [1, 5, 16, 48, 64, 100])
@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_forward_fused(k, dtype):
    b, T, d = 2, 20, 3
    q, Bm, S, C, D = _q_inputs(b, T, d, k, seed=k, dtype=dtype)
    Dx = D.view(1, 1, d).expand(b, T, d)
    got = K.ssm_forward_fused(*(t.to(DEV) for t in (q, Bm, S, C)), Dx.to(DEV))
    assert got.dtype == dtype
    want = oracle.ssm_forward_reference(up(q), up(Bm), up(S), up(C), up(Dx))
    assert_close(got, want, tol(dtype), f"ssm_q k={k} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_forward_fused_wide(dtype):
    """d_inner 2048 at batch 4: the launcher's block size is capped where the
    materialised-q kernel would spill (several rounds of blocks)."""
    b, T, d, k = 4, 9, 2048, 64
    q, Bm, S, C, D = _q_inputs(b, T, d, k, seed=40, dtype=dtype)
    Dx = D.view(1, 1, d).expand(b, T, d)
    got = K.ssm_forward_fused(*(t.to(DEV) for t in (q, Bm, S, C)), Dx.to(DEV))
    want = oracle.ssm_forward_reference(up(q), up(Bm), up(S), up(C), up(Dx))
    assert_close(got, want, tol(dtype), f"ssm_q wide {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_q_empty_walk_writes_state(dtype):
    """mqc_ssm_q_fwd with seq_len 0 and an h_last buffer: h_last = h0, or zeros
    without h0; the per-step operands may be NULL."""
    from mambaqc_amd import _native as nat
    b, d, k = 3, 7, 8
    h0 = rnd(b, d, k, 4, seed=50, dtype=dtype).to(DEV)
    lib = nat.load()
    st = nat.stream_of(h0)
    for src in (h0, None):
        hl = torch.full_like(h0, 7.0)
        rc = lib.mqc_ssm_q_fwd(None, None, None, None, None, 0, 0, 1, nat.ptr(src), None,
                               hl.data_ptr(), b, 0, d, k, nat.dtype_code(h0), st)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(hl, h0 if src is not None else torch.zeros_like(h0))


def test_ssm_forward_fused_strided_D():
    b, T, d, k = 2, 9, 4, 8
    q, Bm, S, C, _ = _q_inputs(b, T, d, k, seed=21, dtype=torch.float32)
    D = rnd(T, b, d, seed=22).transpose(0, 1)           # non-contiguous [b, T, d]
    got = K.ssm_forward_fused(*(t.to(DEV) for t in (q, Bm, S, C)), D.to(DEV))
    want = oracle.ssm_forward_reference(up(q), up(Bm), up(S), up(C), up(D))
    assert_close(got, want, 1e-4, "ssm_q strided D")


@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_step_fused(dtype):
    b, d, k = 3, 5, 16
    q, Bm, S, C, _ = _q_inputs(b, 1, d, k, seed=31, dtype=dtype)
    q, Bm, S, C = q[:, 0], Bm[:, 0], S[:, 0], C[:, 0]
    D = rnd(b, d, seed=32, dtype=dtype)
    h = rnd(b, d, k, 4, seed=33, dtype=dtype)
    h_new, y = K.ssm_step_fused(*(t.to(DEV) for t in (q, Bm, S, C, D, h)))
    h_ref, y_ref = oracle.ssm_step_reference(up(q), up(Bm), up(S), up(C), up(D), up(h))
    assert_close(h_new, h_ref, tol(dtype), "step h")
    assert_close(y, y_ref, tol(dtype), "step y")


# ---------------------------------------------------------------- SSM (block form)
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
    return delta, s, Bm, C, la, li, D


@pytest.mark.parametrize("shape", [(1, 64, 8, 64), (2, 33, 5, 16), (1, 17, 3, 1), (2, 10, 4, 3),
                                   (1, 12, 2, 100), (1, 9, 130, 2),
                                   # block counts that are (2 x 8 = 16, 4 x 12 = 48) and are not
                                   # (3 x 13 = 39) multiples of the 8 XCDs: the remapped and the
                                   # hardware block order
                                   (2, 37, 64, 64), (4, 19, 96, 64), (3, 21, 100, 64),
                                   # enough (b, d) for several states per lane in 16-bit storage
                                   # (two, or four for the inference walk); d ragged;
                                   # walks shorter than, equal to and past one group of 8
                                   # prefetched steps (a tail of 5)
                                   (8, 5, 768, 64), (3, 7, 2050, 64), (8, 8, 768, 64),
                                   (8, 21, 768, 64),
                                   # four states per lane with lanes past d_state (48 of 64),
                                   # and with a 4-lane group (d_state 16)
                                   (8, 9, 1024, 48), (16, 5, 1536, 16)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_fused_dl(shape, dtype):
    a = _dl_inputs(*shape, seed=sum(shape), dtype=dtype)
    got = K.ssm_forward_fused_dl(*(t.to(DEV) for t in a))
    want = oracle.ssm_forward_dl_reference(*(up(t) for t in a))
    assert_close(got, want, tol(dtype), f"ssm_dl {shape} {dtype}")


@pytest.mark.parametrize("shape", [(2, 37, 48), (1, 5, 3), (3, 1, 1), (4, 64, 1536)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_front(shape, dtype):
    """delta = softplus(dt_raw), s = sigmoid(g_raw) * x against float64 torch on
    the same rounded inputs; dt_raw spans torch's softplus threshold (20), and
    known answers pin softplus(0) = log 2, softplus(25) = 25 and s = x / 2 at
    g_raw = 0."""
    g = torch.Generator().manual_seed(sum(shape))
    dt = (torch.randn(*shape, generator=g) * 8).to(dtype)
    gr = (torch.randn(*shape, generator=g) * 4).to(dtype)
    x = torch.randn(*shape, generator=g).to(dtype)
    flat_dt, flat_g = dt.view(-1), gr.view(-1)
    flat_dt[0] = 0.0
    flat_g[0] = 0.0
    if flat_dt.numel() > 2:
        flat_dt[1], flat_dt[2] = 25.0, -30.0
    delta, sv = K.ssm_front(dt.to(DEV), gr.to(DEV), x.to(DEV))
    assert delta.dtype == dtype and sv.dtype == dtype
    want_d = torch.nn.functional.softplus(dt.double())
    want_s = torch.sigmoid(gr.double()) * x.double()
    assert_close(delta, want_d, tol(dtype), f"delta {shape} {dtype}")
    assert_close(sv, want_s, tol(dtype), f"s {shape} {dtype}")
    if dtype == torch.float32:
        # Relative accuracy everywhere, also where softplus(v) ~ exp(v) is tiny.
        rel = ((delta.cpu().double() - want_d).abs() / want_d.abs()).max().item()
        assert rel < 2e-5, rel
    r = 1e-6 if dtype == torch.float32 else 4e-3
    assert abs(delta.view(-1)[0].item() - np.log(2.0)) <= r
    assert abs(sv.view(-1)[0].item() - x.view(-1)[0].item() / 2) <= r * (1 + abs(x.view(-1)[0].item()))
    if flat_dt.numel() > 2:
        assert delta.view(-1)[1].item() == 25.0


def test_ssm_front_unaligned_views():
    """Odd-offset views take the element-wise path and give the same values."""
    base = torch.randn(3, 1 + 2 * 5 * 7, device=DEV)
    dt, gr, x = (base[i, 1:].view(2, 5, 7) for i in range(3))
    d1, s1 = K.ssm_front(dt, gr, x)
    d2, s2 = K.ssm_front(dt.contiguous(), gr.contiguous(), x.contiguous())
    assert torch.equal(d1, d2) and torch.equal(s1, s2)


@pytest.mark.parametrize("shape,dtype,small", [((2, 40, 6, 64), torch.float32, False),
                                               # several states per lane (2 in fp32, 4 in bf16)
                                               ((8, 20, 768, 64), torch.float32, False),
                                               ((8, 20, 768, 64), torch.bfloat16, False),
                                               # long walks with slow decay in 16-bit storage
                                               ((2, 300, 64, 64), torch.bfloat16, True),
                                               ((2, 300, 64, 64), torch.float16, True),
                                               ((8, 260, 768, 64), torch.bfloat16, True)])
def test_ssm_fused_dl_state_carry(shape, dtype, small):
    """Running [0, T) equals running it in pieces from the carried state, bit
    for bit in every storage dtype: the state crosses the call boundary in
    fp32, the precision the walk carries it in. The `small` cases take steps
    delta ~ 0.01 (|q| within about 1 % of 1), where a state rounded to 16 bits
    at every boundary (a recurrent decode) would drift by about 1/(1 - |q|)
    times its rounding error; pieces include single steps."""
    a = _dl_inputs(*shape, seed=41, dtype=dtype)
    if small:
        a = (a[0].float().mul(0.08).to(dtype),) + a[1:]
    dev = [t.to(DEV) for t in a]
    delta, s, Bm, C, la, li, D = dev
    T = shape[1]
    # Whole walks (no time chunks) everywhere: the same arithmetic step by step.
    whole = dict(chunk_len=1 << 30)
    y_full, h_full = K.ssm_forward_fused_dl(*dev, return_state=True, **whole)
    assert h_full.dtype == torch.float32
    cuts = [0, 15, 16, 17, T // 2, T] if T > 40 else [0, 15, T]
    h, ys = None, []
    for t0, t1 in zip(cuts[:-1], cuts[1:]):
        y, h = K.ssm_forward_fused_dl(delta[:, t0:t1], s[:, t0:t1], Bm[:, t0:t1], C[:, t0:t1],
                                      la, li, D, h0=h, return_state=True, **whole)
        ys.append(y)
    assert torch.equal(torch.cat(ys, 1), y_full), "pieces differ from the whole walk"
    assert torch.equal(h, h_full), "final state of the pieces differs"
    # The library's own choice (time chunks where the batch is small) agrees
    # to rounding.
    y_auto, h_auto = K.ssm_forward_fused_dl(*dev, return_state=True)
    assert_close(y_auto, y_full, tol(dtype), "auto walk vs whole walk")
    assert_close(h_auto, h_full, 1e-4, "auto walk state vs whole walk")
    ref_y, ref_h = oracle.ssm_forward_dl_reference(*(up(t) for t in a), return_state=True)
    assert_close(y_full, ref_y, tol(dtype), "y vs oracle")
    # The state is fp32 at every dtype: compare it at the fp32 tolerance where
    # the operands were fp32, at the 16-bit one otherwise (inputs rounded).
    assert_close(h_full, ref_h, tol(dtype), "final state vs oracle")


def test_ssm_fused_dl_config3_full_size():
    """B4 T2048 D1536 S64 bf16 (config 3 sizes). Lanes are independent, so
    d-slices of the full-size output are checked against the oracle on the
    same bf16 inputs. Every lane is checked through linearity in s: with q and
    B fixed, h and the skip term are linear in s, so y(2s) = 2 y(s)."""
    b, T, d, k = 4, 2048, 1536, 64
    g = torch.Generator(device=DEV).manual_seed(0)
    bf = torch.bfloat16
    x = torch.randn(b, T, d, generator=g, device=DEV)
    delta = torch.nn.functional.softplus(torch.randn(b, T, d, generator=g, device=DEV) - 2).to(bf)
    Bm = (torch.randn(b, T, d, k, 4, generator=g, device=DEV, dtype=bf) * 0.02)
    C = (torch.randn(b, T, d, k, 4, generator=g, device=DEV, dtype=bf) * 0.02)
    la = torch.randn(d, k, generator=g, device=DEV) * 0.5 + 1
    li = torch.randn(d, k, 3, generator=g, device=DEV) * 0.1
    D = torch.ones(d, device=DEV)
    s = x.to(bf)
    y = K.ssm_forward_fused_dl(delta, s, Bm, C, la, li, D)
    y2 = K.ssm_forward_fused_dl(delta, (2 * s.float()).to(bf), Bm, C, la, li, D)
    assert_close(y2.float(), 2 * y.float(), 2e-2, "linearity in s")
    # Slices at both ends and in the middle of the grid, in every batch row
    # (each (b, d-block) is its own workgroup).
    for b0, ds in ((0, slice(0, 3)), (1, slice(380, 383)), (2, slice(766, 769)),
                   (3, slice(1150, 1153)), (0, slice(767, 768)), (3, slice(1533, 1536))):
        want = oracle.ssm_forward_dl_reference(
            up(delta[b0:b0 + 1, :, ds]), up(s[b0:b0 + 1, :, ds]), up(Bm[b0:b0 + 1, :, ds]),
            up(C[b0:b0 + 1, :, ds]), up(la[ds]), up(li[ds]), up(D[ds]))
        assert_close(y[b0:b0 + 1, :, ds], want, 2e-2, f"C3 slice b={b0} d={ds}")


# ---------------------------------------------------------------- QLN
def test_qln_golden():
    d = np.load(GOLDEN / "qln.npz")
    q, g, bt = (torch.from_numpy(d[k]) for k in ("q", "gamma", "beta"))
    got = K.quaternion_layer_norm_fused(q.to(DEV), g.to(DEV), bt.to(DEV), eps=float(d["eps"]))
    assert_close(got, torch.from_numpy(d["out"]), 1e-4, "qln golden")


@pytest.mark.parametrize("dm", [1, 7, 64, 130, 1536, 2100, 5000])
@pytest.mark.parametrize("dtype", DTYPES)
def test_qln(dm, dtype):
    q = rnd(2, 3, dm, 4, seed=dm, dtype=dtype)
    gamma = rnd(dm, seed=dm + 1).abs() + 0.5
    beta = rnd(dm, 4, seed=dm + 2) * 0.1
    got, mean, rstd = K.quaternion_layer_norm_fused(q.to(DEV), gamma.to(DEV), beta.to(DEV),
                                                    return_stats=True)
    want = oracle.qln_reference(up(q), up(gamma), up(beta))
    assert_close(got, want, tol(dtype), f"qln d={dm} {dtype}")
    n = torch.sqrt((up(q) ** 2).sum(-1) + 1e-5)
    assert_close(mean, n.mean(-1), 1e-4, "qln mean")
    assert_close(rstd, 1 / torch.sqrt(n.var(-1, unbiased=False) + 1e-5), 1e-3, "qln rstd")


def test_qln_module():
    m = K.QuaternionLayerNorm(24).to(DEV)
    q = rnd(2, 5, 24, 4, seed=51).to(DEV)
    assert_close(m(q), oracle.qln_reference(q.cpu(), m.gamma.detach().cpu(), m.beta.detach().cpu()),
                 1e-4, "qln module")


# ---------------------------------------------------------------- output step
@pytest.mark.parametrize("dtype", DTYPES)
def test_out_gate(dtype):
    rows, dm, di = 37, 24, 48
    x = rnd(rows, dm, seed=61, dtype=dtype)
    xz = rnd(rows, 2 * di, seed=62, dtype=dtype)
    yr = rnd(rows, dm, seed=63, dtype=dtype)
    z = xz.to(DEV).chunk(2, dim=-1)[1]
    got = mambaqc_amd.out_gate(x.to(DEV), z, yr.to(DEV))
    zz = up(xz)[:, di:di + dm]
    assert_close(got, up(x) + torch.sigmoid(zz) * up(yr), tol(dtype), f"out_gate {dtype}")


# ---------------------------------------------------------------- block
def test_block_golden_s1e1():
    d = np.load(GOLDEN / "block_s1e1.npz")
    blk = mambaqc_amd.QuaternionMamba2Block(16, d_state=1, d_conv=4, expand_factor=1)
    blk.load_state_dict({k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p:")})
    blk = blk.to(DEV)
    with torch.no_grad():
        got = blk(torch.from_numpy(d["x"]).to(DEV))
    assert_close(got, torch.from_numpy(d["out"]), 1e-4, "block golden")


def test_block_config1_vs_oracle():
    torch.manual_seed(0)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    x = torch.randn(1, 64, 64)
    want = oracle.block_forward_reference(blk.state_dict(), x, d_state=16)
    with torch.no_grad():
        got = blk.to(DEV)(x.to(DEV))
    assert_close(got, want, 1e-4, "block C1 fp32")


def test_block_bf16_vs_oracle():
    torch.manual_seed(1)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    blk = blk.to(torch.bfloat16)
    x = torch.randn(2, 48, 64).to(torch.bfloat16)
    sd = {k: v.float() for k, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.float(), d_state=16)
    with torch.no_grad():
        got = blk.to(DEV)(x.to(DEV))
    assert got.dtype == torch.bfloat16
    assert_close(got, want, 2e-2, "block bf16")


def test_block_headline_width_bf16_vs_oracle():
    """The headline configuration's block (d_model 768, d_state 64, expand 2:
    d_inner 1536) in bf16 at B4 T256 against the oracle in fp32 on the same
    bf16-rounded weights and input, on both of its inference paths: the default
    (256 tokens per sequence and 1024 token rows: the B/C projections fused into
    the SSM kernel, and the output step as one kernel, as the benchmark times) and
    the unfused one (wide_linear's column blocks of 1.2 GB of weight each, the
    inference walk with four states per lane, out_proj then the gate kernel)."""
    from mambaqc_amd.layers import quaternion_linear as ql

    torch.manual_seed(11)
    with torch.device(DEV):
        blk = mambaqc_amd.QuaternionMamba2Block(768, d_state=64, d_conv=4, expand_factor=2)
    blk = blk.to(torch.bfloat16)
    x = torch.randn(4, 256, 768, generator=torch.Generator(device=DEV).manual_seed(12),
                    device=DEV).to(torch.bfloat16)
    n, k = blk.B_proj.weight.shape
    assert len(ql._blocks(n, k, 2)) > 1 and x.numel() // 768 >= ql.WIDE_LINEAR_MIN_ROWS
    x_act = torch.empty(4, 256, blk.d_inner, device=DEV, dtype=torch.bfloat16)
    assert blk._use_fused_bc(x_act)
    with torch.no_grad():
        got = blk(x)
        blk.fuse_bc = blk.fuse_out = False
        got_unfused = blk(x)
    assert got.dtype == torch.bfloat16
    sd = {kk: v.detach().float().cpu() for kk, v in blk.state_dict().items()}
    want = oracle.block_forward_reference(sd, x.float().cpu(), d_state=64)
    assert_close(got, want, 2e-2, "block d768 s64 e2 bf16 (fused paths)")
    assert_close(got_unfused, want, 2e-2, "block d768 s64 e2 bf16 (unfused)")


def test_block_built_under_inference_mode():
    """A bf16 block whose parameters are inference tensors (built inside
    torch.inference_mode) gives the same output as one built normally; its
    parameter conversions cannot be cached and are redone every call."""
    torch.manual_seed(3)
    ref_blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16).to(DEV, torch.bfloat16)
    x = torch.randn(2, 20, 64, device=DEV).to(torch.bfloat16)
    with torch.inference_mode():
        torch.manual_seed(3)
        blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16).to(DEV, torch.bfloat16)
        assert blk.Lambda_alpha.is_inference()
        got = blk(x)
        got2 = blk(x)
        want = ref_blk(x)
    assert torch.equal(got, want) and torch.equal(got2, want)


# ---------------------------------------------------------------- front of block
def _conv_silu_ref(x, w, b):
    """silu(CausalConv1d(x)) in float64 (layers/causal_conv1d.py:68-91 + F.silu)."""
    C, _, K = w.shape
    xt = torch.nn.functional.pad(x.double().transpose(1, 2), (K - 1, 0))
    pre = torch.nn.functional.conv1d(xt, w.double(), None if b is None else b.double(), groups=C)
    return torch.nn.functional.silu(pre).transpose(1, 2)


@pytest.mark.parametrize("shape", [(2, 37, 48, 4), (1, 3, 16, 4), (2, 20, 13, 3), (1, 50, 24, 1),
                                   (3, 17, 64, 6)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_causal_conv_silu(shape, dtype):
    from mambaqc_amd.layers.causal_conv1d import causal_conv1d_silu
    b, T, C, K = shape
    g = torch.Generator().manual_seed(sum(shape))
    xz = torch.randn(b, T, 2 * C, generator=g).to(dtype)
    w = torch.randn(C, 1, K, generator=g) * 0.5
    bias = torch.randn(C, generator=g) * 0.1
    x_in = xz.to(DEV).chunk(2, dim=-1)[0]                 # strided view, row stride 2C
    got = causal_conv1d_silu(x_in, w.to(DEV), bias.to(DEV))
    assert got.is_contiguous() and got.dtype == dtype
    assert_close(got, _conv_silu_ref(xz[..., :C], w, bias), tol(dtype), f"conv_silu {shape} {dtype}")


def test_causal_conv_silu_long_runs():
    """A launch large enough for 16-step runs per thread (the small shapes above
    take 4-step runs): B12 T2048 C1536 bf16 against torch's fp32 conv + SiLU on
    the same rounded input."""
    from mambaqc_amd.layers.causal_conv1d import causal_conv1d_silu
    b, T, C, K = 12, 2048, 1536, 4
    g = torch.Generator(device=DEV).manual_seed(5)
    xz = torch.randn(b, T, 2 * C, generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn(C, 1, K, generator=g, device=DEV) * 0.5
    bias = torch.randn(C, generator=g, device=DEV) * 0.1
    x_in = xz.chunk(2, dim=-1)[0]
    got = causal_conv1d_silu(x_in, w, bias)
    xt = torch.nn.functional.pad(x_in.float().transpose(1, 2), (K - 1, 0))
    want = torch.nn.functional.silu(
        torch.nn.functional.conv1d(xt, w, bias, groups=C)).transpose(1, 2)
    assert_close(got, want, 2e-2, "conv_silu long runs")


# ---------------------------------------------------------------- wide projections
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1000, 4096, 777])
def test_wide_linear_column_blocks(monkeypatch, dtype, n):
    """wide_linear's column-block GEMMs (forced here with a 64 KiB weight bound,
    so N = 777 splits into ragged blocks) equal one fp64 product, and the
    block's B/C projections take that path under no_grad."""
    from mambaqc_amd.layers import quaternion_linear as ql

    monkeypatch.setattr(ql, "WIDE_LINEAR_CHUNK_BYTES", 64 << 10)
    monkeypatch.setattr(ql, "WIDE_LINEAR_MIN_ROWS", 1)
    x = rnd(3, 5, 96, seed=1, dtype=dtype).to(DEV)
    w = rnd(n, 96, seed=2, dtype=dtype, scale=0.1).to(DEV)
    with torch.no_grad():
        got = ql.wide_linear(x, w)
    assert got.shape == (3, 5, n) and got.dtype == dtype
    assert_close(got, up(x) @ up(w).t(), tol(dtype), f"wide_linear {dtype} n={n}")

    lin = ql.real_to_quaternion_projection(96, n // 4 if n % 4 == 0 else 250, bias=True)
    lin = lin.to(DEV, dtype)
    with torch.no_grad():
        lin.bias.normal_()
        out = lin(x)
    want = (up(x) @ up(lin.weight).t()).view(3, 5, -1, 4) + up(lin.bias)
    assert_close(out, want, tol(dtype), f"real->quaternion projection {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [777, 769, 4096])
def test_wide_linear_backward(monkeypatch, dtype, n):
    """Gradients of the blocked GEMMs (row-block dW, K-block dx with fp32
    partials) against fp64 products, with ragged blocks: dx from one batched
    GEMM over equal row blocks where a block count divides n (777: 21 blocks
    of 37 rows; 4096: 16 of 256), from one GEMM per block where none does
    (769, a prime)."""
    from mambaqc_amd.layers import quaternion_linear as ql

    monkeypatch.setattr(ql, "WIDE_LINEAR_CHUNK_BYTES", 16 << 10)
    monkeypatch.setattr(ql, "WIDE_LINEAR_MIN_ROWS", 1)
    x = rnd(2, 9, 96, seed=5, dtype=dtype).to(DEV).requires_grad_()
    w = rnd(n, 96, seed=6, dtype=dtype, scale=0.1).to(DEV).requires_grad_()
    gy = rnd(2, 9, n, seed=7, dtype=dtype).to(DEV)
    y = ql.wide_linear(x, w)
    assert y.grad_fn is not None and len(ql._blocks(n, 96, w.element_size())) > 1
    assert (ql._dx_batches(n, 96, w.element_size()) > 0) == (n != 769)
    y.backward(gy)
    assert_close(y, up(x) @ up(w).t(), tol(dtype), "y")
    assert_close(x.grad, up(gy) @ up(w), tol(dtype), "dx")
    assert_close(w.grad, up(gy).reshape(-1, n).t() @ up(x).reshape(-1, 96), tol(dtype), "dW")


def test_wide_linear_autocast_matches_f_linear(monkeypatch):
    """Under fp16 autocast the blocked path gives F.linear's dtypes and, within
    fp16 rounding, its values and gradients (fp32 weight, fp32 input)."""
    from mambaqc_amd.layers import quaternion_linear as ql

    monkeypatch.setattr(ql, "WIDE_LINEAR_CHUNK_BYTES", 16 << 10)
    monkeypatch.setattr(ql, "WIDE_LINEAR_MIN_ROWS", 1)
    x = rnd(3, 7, 64, seed=8).to(DEV)
    w = rnd(520, 64, seed=9, scale=0.1).to(DEV)
    outs = []
    for fn in (ql.wide_linear, torch.nn.functional.linear):
        xi = x.clone().requires_grad_()
        wi = w.clone().requires_grad_()
        with torch.autocast("cuda", dtype=torch.float16):
            y = fn(xi, wi)
        assert y.dtype == torch.float16
        (y.float() ** 2).sum().backward()
        assert xi.grad.dtype == torch.float32 and wi.grad.dtype == torch.float32
        outs.append((y, xi.grad, wi.grad))
    for a, b, what in zip(outs[0], outs[1], ("y", "dx", "dW")):
        assert_close(a, b, 2e-2, f"autocast {what}")


def test_wide_linear_records_autograd(monkeypatch):
    """With autograd recording, the blocked path records a backward node and
    its weight gradient is right (fp32, a sum over rows)."""
    from mambaqc_amd.layers import quaternion_linear as ql

    monkeypatch.setattr(ql, "WIDE_LINEAR_CHUNK_BYTES", 1 << 10)
    monkeypatch.setattr(ql, "WIDE_LINEAR_MIN_ROWS", 1)
    x = rnd(4, 32, seed=3).to(DEV).requires_grad_()
    w = rnd(64, 32, seed=4).to(DEV).requires_grad_()
    y = ql.wide_linear(x, w)
    assert y.grad_fn is not None
    y.sum().backward()
    assert_close(w.grad, up(x).sum(0, keepdim=True).expand(64, 32), 1e-4, "dW")
