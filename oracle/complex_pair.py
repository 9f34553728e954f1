"""An independent oracle for the block's SSM via H = C_u (+) C_u m — TEST ONLY.

For a fixed Lambda = (a, v) with unit axis u = v/|v|, every Cayley step
q_t = Cayley(delta_t Lambda) lies in span{1, u}, which is a copy of C (u -> i).
Pick a unit pure m orthogonal to u and w = u x m = u (x) m. In the orthonormal
basis {1, u, m, w} a quaternion h = c0 + c1 u + c2 m + c3 w splits as
h1 = c0 + i c1, h2 = c2 + i c3 with h = h1 + h2 (x) m, and left
multiplication by q = x + y u acts as the complex number x + i y on both h1
and h2. The Cayley map is the complex one, (1 + zeta/2) / (1 - zeta/2) with
zeta = delta (a + i |v|). The recurrence h_t = q_t h_{t-1} + s_t B_t then runs
as two complex scalar recurrences per (b, d, k), and y_t = sum_k L(C) h_t is
formed with an explicit 4x4 left-multiplication matrix.

None of oracle/quat.py is used here: this pins ssm_forward_dl_reference (its
Cayley, Hamilton product, Lambda and recurrence) by a separate derivation.
Valid while |1 - z/2|^2 > eps (the clamp never engages).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _left_matrix(p: torch.Tensor) -> torch.Tensor:
    """L(p) with p (x) q = L(p) q, as [..., 4, 4]."""
    p0, p1, p2, p3 = p.unbind(-1)
    rows = [
        torch.stack((p0, -p1, -p2, -p3), -1),
        torch.stack((p1, p0, -p3, p2), -1),
        torch.stack((p2, p3, p0, -p1), -1),
        torch.stack((p3, -p2, p1, p0), -1),
    ]
    return torch.stack(rows, -2)


def _basis(v: torch.Tensor) -> torch.Tensor:
    """Orthonormal [..., 4, 4] with columns (1, u, m, w) for vector parts v [..., 3]."""
    r = v.norm(dim=-1, keepdim=True)
    ex = torch.tensor([1.0, 0.0, 0.0], dtype=v.dtype).expand_as(v)
    u = torch.where(r > 0, v / r.clamp_min(1e-300), ex)
    ey = torch.tensor([0.0, 1.0, 0.0], dtype=v.dtype).expand_as(v)
    e = torch.where(u[..., :1].abs() < 0.9, ex, ey)
    m = e - (e * u).sum(-1, keepdim=True) * u
    m = m / m.norm(dim=-1, keepdim=True)
    w = torch.linalg.cross(u, m, dim=-1)
    zero = torch.zeros_like(r)
    cols = [
        torch.cat((torch.ones_like(r), torch.zeros_like(v)), -1),
        torch.cat((zero, u), -1),
        torch.cat((zero, m), -1),
        torch.cat((zero, w), -1),
    ]
    return torch.stack(cols, -1)


def ssm_forward_complex(delta, s, B, C, lambda_alpha, lambda_imag, D):
    """Same contract as oracle.ssm_forward_dl_reference (no h0). Computes in float64."""
    f64 = torch.float64
    delta, s, B, C = (t.detach().cpu().to(f64) for t in (delta, s, B, C))
    la, li, D = (t.detach().cpu().to(f64) for t in (lambda_alpha, lambda_imag, D))
    b, T, d, k, _ = B.shape
    a = -F.softplus(la)                      # [d, k]
    v = torch.tanh(li)                       # [d, k, 3]
    P = _basis(v)                            # [d, k, 4, 4]
    Pt = P.transpose(-1, -2)
    rad = v.norm(dim=-1)                     # [d, k]
    h1 = torch.zeros(b, d, k, dtype=torch.complex128)
    h2 = torch.zeros(b, d, k, dtype=torch.complex128)
    y = torch.empty(b, T, d, 4, dtype=f64)
    for t in range(T):
        zeta = delta[:, t, :, None] * torch.complex(a, rad)[None]
        lam = (1 + zeta / 2) / (1 - zeta / 2)
        cb = (Pt[None] @ B[:, t, ..., None])[..., 0]        # [b, d, k, 4]
        st = s[:, t, :, None]
        h1 = lam * h1 + st * torch.complex(cb[..., 0], cb[..., 1])
        h2 = lam * h2 + st * torch.complex(cb[..., 2], cb[..., 3])
        coords = torch.stack((h1.real, h1.imag, h2.real, h2.imag), -1)
        h = (P[None] @ coords[..., None])[..., 0]           # [b, d, k, 4]
        yt = (_left_matrix(C[:, t]) @ h[..., None])[..., 0].sum(dim=2)
        yt[..., 0] += D[None] * s[:, t]
        y[:, t] = yt
    return y
