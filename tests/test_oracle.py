"""Pins of the CPU oracle (oracle/) — every function is checked by something
other than its own formula: the reference's golden fixtures (written from the
reference's CPU code by tests/golden/make_golden.py), known answers from the
quaternion multiplication table, closed forms, an independent complex-pair
derivation of the SSM, and brute force on tiny inputs. The reference's own
property tests (mambaqc/tests/test_quaternion_ops.py:33-269) are ported here
against the oracle.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN

torch.set_default_dtype(torch.float32)


def qt(*v, dtype=torch.float64):
    return torch.tensor(v, dtype=dtype)


# ---------------------------------------------------------------- Hamilton product
BASIS = {"1": qt(1, 0, 0, 0), "i": qt(0, 1, 0, 0), "j": qt(0, 0, 1, 0), "k": qt(0, 0, 0, 1)}
# Hamilton's table: i^2 = j^2 = k^2 = ijk = -1.
TABLE = {
    ("i", "j"): ("k", 1), ("j", "i"): ("k", -1),
    ("j", "k"): ("i", 1), ("k", "j"): ("i", -1),
    ("k", "i"): ("j", 1), ("i", "k"): ("j", -1),
    ("i", "i"): ("1", -1), ("j", "j"): ("1", -1), ("k", "k"): ("1", -1),
}


def test_hamilton_multiplication_table():
    for a in "1ijk":
        for b in "1ijk":
            if a == "1":
                want = BASIS[b]
            elif b == "1":
                want = BASIS[a]
            else:
                name, sign = TABLE[(a, b)]
                want = sign * BASIS[name]
            assert torch.equal(oracle.hamilton(BASIS[a], BASIS[b]), want), (a, b)


def test_hamilton_bilinear_brute_force():
    # Expand p and q over the basis and sum the table products term by term.
    g = torch.Generator().manual_seed(3)
    p = torch.randn(20, 4, generator=g, dtype=torch.float64)
    q = torch.randn(20, 4, generator=g, dtype=torch.float64)
    names = "1ijk"
    want = torch.zeros(20, 4, dtype=torch.float64)
    for a in range(4):
        for b in range(4):
            prod = oracle.hamilton(BASIS[names[a]], BASIS[names[b]])
            want += (p[:, a] * q[:, b])[:, None] * prod
    torch.testing.assert_close(oracle.hamilton(p, q), want, rtol=1e-12, atol=1e-12)


def test_hamilton_known_pairs():
    # The reference's non-commutativity pair (test_quaternion_ops.py:85-94).
    p, q = qt(1, 1, 0, 0), qt(1, 0, 1, 0)
    assert torch.equal(oracle.hamilton(p, q), qt(1, 1, 1, 1))
    assert torch.equal(oracle.hamilton(q, p), qt(1, 1, 1, -1))


class TestReferenceProperties:
    """mambaqc/tests/test_quaternion_ops.py:33-191 against the oracle."""

    def test_identity(self):
        q = torch.randn(10, 4)
        assert torch.allclose(oracle.hamilton(q, torch.tensor([1.0, 0, 0, 0]).expand_as(q)), q, atol=1e-6)

    def test_conjugate_product(self):
        q = torch.randn(10, 4)
        r = oracle.hamilton(q, oracle.conjugate(q))
        want = torch.cat([(q ** 2).sum(-1, keepdim=True), torch.zeros(10, 3)], -1)
        assert torch.allclose(r, want, atol=1e-5)

    def test_inverse(self):
        q = torch.randn(10, 4) + 0.5
        r = oracle.hamilton(q, oracle.inverse(q))
        assert torch.allclose(r, torch.tensor([1.0, 0, 0, 0]).expand_as(r), atol=1e-5)

    def test_associativity(self):
        p, q, r = torch.randn(3, 5, 4).unbind(0)
        assert torch.allclose(oracle.hamilton(oracle.hamilton(p, q), r),
                              oracle.hamilton(p, oracle.hamilton(q, r)), atol=1e-5)

    def test_norm_multiplicativity(self):
        p, q = torch.randn(2, 10, 4).unbind(0)
        assert torch.allclose(oracle.norm(oracle.hamilton(p, q)), oracle.norm(p) * oracle.norm(q), rtol=1e-5)

    def test_conjugate_involution_and_parts(self):
        q = torch.randn(10, 4)
        c = oracle.conjugate(q)
        assert torch.allclose(oracle.conjugate(c), q, atol=1e-6)
        assert torch.allclose(q[:, 0], c[:, 0]) and torch.allclose(q[:, 1:], -c[:, 1:])

    def test_inverse_twice_and_norm(self):
        q = torch.randn(10, 4) + 1.0
        assert torch.allclose(oracle.inverse(oracle.inverse(q)), q, atol=1e-5)
        assert torch.allclose(oracle.norm(oracle.inverse(q)), 1.0 / oracle.norm(q), rtol=1e-5)
        assert torch.allclose(oracle.inverse(torch.tensor([[1.0, 0, 0, 0]])), torch.tensor([[1.0, 0, 0, 0]]))

    def test_norm_values(self):
        assert (oracle.norm(torch.randn(100, 4)) >= 0).all()
        assert oracle.norm(torch.tensor([[1.0, 0, 0, 0]])).item() == 1.0
        assert oracle.norm(torch.zeros(1, 4)).item() == 0.0

    def test_inverse_clamp(self):
        # |q|^2 below eps: conj(q) / eps (quaternion_ops.py:409).
        q = qt(1e-4, 0, 0, 0)
        assert torch.allclose(oracle.inverse(q, eps=1e-6), qt(1e-4 / 1e-6, 0, 0, 0))


# ---------------------------------------------------------------- Cayley
def test_cayley_golden():
    d = np.load(GOLDEN / "cayley.npz")
    got = oracle.cayley_reference(torch.from_numpy(d["z"]), eps=float(d["eps"]))
    assert torch.equal(got, torch.from_numpy(d["q"]))


def test_cayley_zero_is_identity():
    q = oracle.cayley_reference(torch.zeros(2, 4, 8, 16, 4))
    want = torch.zeros_like(q)
    want[..., 0] = 1
    assert torch.allclose(q, want, atol=1e-5)


def test_cayley_real_axis_closed_form():
    a = torch.linspace(-5, 1.5, 27, dtype=torch.float64)
    z = torch.zeros(1, 1, 1, 27, 4, dtype=torch.float64)
    z[..., 0] = a
    q = oracle.cayley_reference(z)
    torch.testing.assert_close(q[..., 0].reshape(-1), (1 + a / 2) / (1 - a / 2))
    assert (q[..., 1:] == 0).all()


def test_cayley_pure_imaginary_is_rotation():
    g = torch.Generator().manual_seed(5)
    v = torch.randn(50, 3, generator=g, dtype=torch.float64) * 2
    z = torch.cat([torch.zeros(50, 1, dtype=torch.float64), v], -1).view(1, 1, 1, 50, 4)
    q = oracle.cayley_reference(z).view(50, 4)
    r = v.norm(dim=-1)
    theta = 2 * torch.atan(r / 2)
    torch.testing.assert_close(q[:, 0], torch.cos(theta))
    torch.testing.assert_close(q[:, 1:], torch.sin(theta)[:, None] * v / r[:, None])


def test_cayley_complex_closed_form_and_stability():
    # In the plane span{1, v}, Cayley is the complex map (1 + zeta/2) / (1 - zeta/2).
    g = torch.Generator().manual_seed(6)
    z = torch.randn(1, 2, 3, 40, 4, generator=g, dtype=torch.float64)
    z[..., 0] = -z[..., 0].abs() - 0.01
    q = oracle.cayley_reference(z)
    r = z[..., 1:].norm(dim=-1)
    lam = (1 + torch.complex(z[..., 0], r) / 2) / (1 - torch.complex(z[..., 0], r) / 2)
    torch.testing.assert_close(q[..., 0], lam.real)
    torch.testing.assert_close(q[..., 1:], (lam.imag / r)[..., None] * z[..., 1:])
    assert (oracle.norm(q) < 1).all()  # Re z < 0 => |q| < 1
    z[..., 0] = 0
    torch.testing.assert_close(oracle.norm(oracle.cayley_reference(z)), torch.ones_like(r))


# ---------------------------------------------------------------- cumulative product
def test_cumprod_order_known_answer():
    i, j = BASIS["i"], BASIS["j"]
    q = torch.stack([i, j]).view(1, 2, 1, 1, 4)
    out = oracle.cumprod_reference(q).view(2, 4)
    assert torch.equal(out[0], i)
    assert torch.equal(out[1], -BASIS["k"])  # j (x) i = -k


def test_cumprod_commuting_axis_closed_form():
    g = torch.Generator().manual_seed(7)
    n = torch.randn(3, 3, generator=g, dtype=torch.float64)
    n = n / n.norm(dim=-1, keepdim=True)
    theta = torch.rand(2, 9, 3, generator=g, dtype=torch.float64)
    q = torch.cat([torch.cos(theta)[..., None], torch.sin(theta)[..., None] * n], -1).unsqueeze(3)
    out = oracle.cumprod_reference(q)
    cs = theta.cumsum(1)
    want = torch.cat([torch.cos(cs)[..., None], torch.sin(cs)[..., None] * n], -1).unsqueeze(3)
    torch.testing.assert_close(out, want)


def test_cumprod_real_is_torch_cumprod():
    g = torch.Generator().manual_seed(8)
    a = torch.randn(2, 11, 3, 2, generator=g, dtype=torch.float64)
    q = torch.zeros(2, 11, 3, 2, 4, dtype=torch.float64)
    q[..., 0] = a
    out = oracle.cumprod_reference(q)
    torch.testing.assert_close(out[..., 0], torch.cumprod(a, dim=1))
    assert (out[..., 1:] == 0).all()


def test_cumprod_brute_force_and_identity():
    # Reference tests :235-269.
    q = torch.randn(1, 8, 4, 8, 4)
    out = oracle.cumprod_reference(q)
    manual = q[:, 0]
    for t in range(1, 8):
        manual = oracle.hamilton(q[:, t], manual)
    assert torch.allclose(out[:, -1], manual, atol=1e-4)
    ident = torch.zeros(2, 10, 8, 16, 4)
    ident[..., 0] = 1
    assert torch.allclose(oracle.cumprod_reference(ident), ident, atol=1e-5)


# ---------------------------------------------------------------- SSM
def _ssm_inputs(b, T, d, k, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=dtype)
    delta = torch.nn.functional.softplus(r(b, T, d) - 1)
    return dict(delta=delta, s=r(b, T, d), B=r(b, T, d, k, 4), C=r(b, T, d, k, 4),
                lambda_alpha=r(d, k) * 0.5 + 1, lambda_imag=r(d, k, 3) * 0.3, D=r(d))


@pytest.mark.parametrize("shape", [(2, 12, 3, 5), (1, 30, 2, 16), (1, 5, 4, 1)])
def test_ssm_dl_matches_complex_pair_oracle(shape):
    a = _ssm_inputs(*shape, seed=sum(shape))
    y1 = oracle.ssm_forward_dl_reference(**a)
    y2 = oracle.ssm_forward_complex(**a)
    torch.testing.assert_close(y1, y2, rtol=1e-10, atol=1e-10)


def test_ssm_zero_input_gives_skip_only():
    b, T, d, k = 2, 6, 3, 4
    g = torch.Generator().manual_seed(9)
    q, C = torch.randn(2, b, T, d, k, 4, generator=g).unbind(0)
    S = torch.randn(b, T, d, 4, generator=g)
    D = torch.randn(b, T, d, generator=g)
    y = oracle.ssm_forward_reference(q, torch.zeros_like(q), S, C, D)
    torch.testing.assert_close(y, D[..., None] * S)


def test_ssm_zero_evolution_is_memoryless():
    b, T, d, k = 2, 5, 3, 4
    g = torch.Generator().manual_seed(10)
    Bm, C = torch.randn(2, b, T, d, k, 4, generator=g).unbind(0)
    S = torch.randn(b, T, d, 4, generator=g)
    D = torch.zeros(b, T, d)
    y = oracle.ssm_forward_reference(torch.zeros_like(Bm), Bm, S, C, D)
    # h_t = B_t (x) S_t ; y_t = sum_k C_t (x) h_t, built from the basis table.
    h = oracle.hamilton(Bm, S.unsqueeze(3))
    torch.testing.assert_close(y, oracle.hamilton(C, h).sum(3))


def test_ssm_real_case_is_scalar_selective_scan():
    b, T, d, k = 1, 9, 2, 3
    g = torch.Generator().manual_seed(11)
    a = torch.rand(b, T, d, k, generator=g, dtype=torch.float64)
    bb = torch.randn(b, T, d, k, generator=g, dtype=torch.float64)
    c = torch.randn(b, T, d, k, generator=g, dtype=torch.float64)
    s = torch.randn(b, T, d, generator=g, dtype=torch.float64)
    Dv = torch.randn(b, T, d, generator=g, dtype=torch.float64)
    emb = lambda x: torch.stack([x, *(torch.zeros_like(x),) * 3], -1)
    y = oracle.ssm_forward_reference(emb(a), emb(bb), emb(s), emb(c), Dv)
    want = torch.zeros(b, T, d, dtype=torch.float64)
    for bi in range(b):
        for di in range(d):
            for ki in range(k):
                h = 0.0
                for t in range(T):
                    h = a[bi, t, di, ki].item() * h + bb[bi, t, di, ki].item() * s[bi, t, di].item()
                    want[bi, t, di] += c[bi, t, di, ki].item() * h
    want += Dv * s
    torch.testing.assert_close(y[..., 0], want)
    assert (y[..., 1:] == 0).all()


def test_ssm_step_chain_equals_forward():
    b, T, d, k = 2, 4, 3, 5
    g = torch.Generator().manual_seed(12)
    q, Bm, C = torch.randn(3, b, T, d, k, 4, generator=g).unbind(0)
    S = torch.randn(b, T, d, 4, generator=g)
    D = torch.randn(b, T, d, generator=g)
    y, h = oracle.ssm_forward_reference(q, Bm, S, C, D, return_state=True)
    h2 = torch.zeros(b, d, k, 4)
    for t in range(T):
        h2, yt = oracle.ssm_step_reference(q[:, t], Bm[:, t], S[:, t], C[:, t], D[:, t], h2)
        torch.testing.assert_close(yt, y[:, t])
    torch.testing.assert_close(h, h2)


# ---------------------------------------------------------------- QLN
def test_qln_golden():
    d = np.load(GOLDEN / "qln.npz")
    got = oracle.qln_reference(torch.from_numpy(d["q"]), torch.from_numpy(d["gamma"]),
                               torch.from_numpy(d["beta"]), eps=float(d["eps"]))
    assert torch.equal(got, torch.from_numpy(d["out"]))


def test_qln_invariants():
    g = torch.Generator().manual_seed(13)
    q = torch.randn(3, 5, 64, 4, generator=g, dtype=torch.float64) * 3
    gamma = torch.rand(64, generator=g, dtype=torch.float64) + 0.5
    beta = torch.randn(64, 4, generator=g, dtype=torch.float64)
    out = oracle.qln_reference(q, gamma, beta, eps=1e-12)
    u = (out - beta) / gamma[:, None]
    nq = q.norm(dim=-1, keepdim=True)
    # Direction preserved: u is parallel to q; the signed scale is the normalised norm.
    signed = (u * q / nq).sum(-1)
    torch.testing.assert_close(u, signed[..., None] * q / nq)
    torch.testing.assert_close(signed.mean(-1), torch.zeros(3, 5, dtype=torch.float64), atol=1e-9, rtol=0)
    torch.testing.assert_close(signed.var(-1, unbiased=False), torch.ones(3, 5, dtype=torch.float64))


# ---------------------------------------------------------------- block
def test_block_golden_s1e1():
    d = np.load(GOLDEN / "block_s1e1.npz")
    sd = {k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p:")}
    got = oracle.block_forward_reference(sd, torch.from_numpy(d["x"]), d_state=1)
    torch.testing.assert_close(got, torch.from_numpy(d["out"]), rtol=1e-6, atol=1e-6)


def test_block_gate_slice_is_identity_at_expand_one():
    # D1 only changes anything when expand_factor > 1: at expand 1 z[..., :d_model] is z.
    d = np.load(GOLDEN / "block_s1e1.npz")
    sd = {k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p:")}
    assert sd["in_proj.weight"].shape[0] == 2 * d["x"].shape[-1]


# ---------------------------------------------------------------- LM
def test_lm_golden_s1e1():
    """oracle.lm_forward_reference against the reference LM's own forward
    (d_state 1, expand 1: the LM configuration its CPU path runs)."""
    d = np.load(GOLDEN / "lm_s1e1.npz")
    sd = {k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p:")}
    logits, loss = oracle.lm_forward_reference(
        sd, torch.from_numpy(d["input_ids"]), n_layers=2, d_state=1, vocab_size=37,
        labels=torch.from_numpy(d["labels"]))
    torch.testing.assert_close(logits, torch.from_numpy(d["logits"]), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(loss, torch.from_numpy(d["loss"]), rtol=1e-5, atol=1e-6)
