"""Pins the second-order oracle (``oracle/udtw_tangent.py``) on the CPU.

The tangent recursions are checked against three things they were not
derived from:
* the reference's stored Hessian of soft-DTW on a cost matrix
  (``parity.second_order``, method ``soft_dtw``), column by column;
* double reverse-mode autograd through the oracle's differentiable form of
  the DP (``dp_value``, a finite-sentinel restatement of the recurrence),
  which differentiates the recurrence mechanically, penalty and band included;
* central finite differences of the oracle's analytic first-order backward.
A dropped term (the penalty's weight derivative, the tangent of the weights
in the backward) or a sign error fails all three.
"""

import pytest
import torch

from oracle import udtw as OU
from oracle.udtw_tangent import dp_tangent

from golden_cases import golden

f64 = dict(dtype=torch.float64)


def _rand(shape, seed, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return shift + scale * torch.rand(shape, generator=g, **f64)


def test_soft_dtw_hessian_matches_reference_golden():
    ref = golden("parity.second_order", method="soft_dtw")
    x, H = ref["x"], ref["hessian"]
    T, U = x.shape
    n = T * U
    C = x.expand(n, T, U).contiguous()
    basis = torch.eye(n, **f64).view(n, T, U)
    z = torch.zeros(n, **f64)
    tC, _, _, _ = dp_tangent(C, torch.zeros_like(C), basis, torch.zeros_like(C),
                             torch.ones(n, **f64), z, z, z, 0.3)
    # column k of the Hessian is the tangent along the k-th unit direction
    torch.testing.assert_close(tC.reshape(n, n).T, H.reshape(n, n), rtol=1e-9, atol=1e-10)


CASES = [  # (B, N, M, gamma, bandwidth)
    (2, 4, 5, 0.7, 0.0),
    (3, 6, 6, 0.4, 2.0),
    (1, 7, 4, 1.3, 0.0),
    (2, 5, 9, 0.25, 4.0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}N{}M{}w{}".format(c[0], c[1], c[2], c[4]))
def test_tangent_equals_double_autograd_through_dp_value(case):
    B, N, M, gamma, band = case
    C = _rand((B, N, M), 1, 2.0).requires_grad_(True)
    Q = _rand((B, N, M), 2, 2.0, -1.0).requires_grad_(True)
    gr = _rand((B,), 3, 2.0, -1.0).requires_grad_(True)
    gp = _rand((B,), 4, 2.0, -1.0).requires_grad_(True)
    vC, vQ = _rand((B, N, M), 5, 2.0, -1.0), _rand((B, N, M), 6, 2.0, -1.0)
    tgr, tgp = _rand((B,), 7, 2.0, -1.0), _rand((B,), 8, 2.0, -1.0)
    r, p = OU.dp_value(C, Q, gamma, band)
    dC, dQ = torch.autograd.grad((gr * r + gp * p).sum(), (C, Q), create_graph=True)
    # d/de of the gradient at (C + e vC, Q + e vQ, gr + e tgr, gp + e tgp)
    hC, hQ, t_r, t_p = torch.autograd.grad((dC * vC).sum() + (dQ * vQ).sum(), (C, Q, gr, gp),
                                           retain_graph=True)
    drC, = torch.autograd.grad(r.sum(), C, retain_graph=True)
    dpC, dpQ = torch.autograd.grad(p.sum(), (C, Q))
    want_c = hC + tgr.view(-1, 1, 1) * drC + tgp.view(-1, 1, 1) * dpC
    want_q = hQ + tgp.view(-1, 1, 1) * dpQ
    got = dp_tangent(C.detach(), Q.detach(), vC, vQ, gr.detach(), gp.detach(), tgr, tgp, gamma,
                     band)
    for g, w in zip(got, (want_c, want_q, t_r, t_p)):
        torch.testing.assert_close(g, w, rtol=1e-10, atol=1e-11)


def test_tangent_equals_finite_differences_of_the_analytic_backward():
    B, N, M, gamma, band = 2, 6, 8, 0.5, 3.0
    C, Q = _rand((B, N, M), 11, 2.0), _rand((B, N, M), 12, 2.0, -1.0)
    vC, vQ = _rand((B, N, M), 13, 2.0, -1.0), _rand((B, N, M), 14, 2.0, -1.0)
    gr, gp = torch.tensor([1.0, -0.5], **f64), torch.tensor([0.75, 2.0], **f64)
    z = torch.zeros(B, **f64)

    def grad_at(e):
        c, q = C + e * vC, Q + e * vQ
        _, _, R, P = OU.dp_forward(c, q, gamma, band)
        return OU.dp_backward(c, q, R, P, gr, gp, gamma)
    h = 1e-5
    (cp, qp), (cm, qm) = grad_at(h), grad_at(-h)
    tC, tQ, _, _ = dp_tangent(C, Q, vC, vQ, gr, gp, z, z, gamma, band)
    torch.testing.assert_close(tC, (cp - cm) / (2 * h), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(tQ, (qp - qm) / (2 * h), rtol=1e-6, atol=1e-7)


def test_hessian_vector_products_are_symmetric():
    """<u, H v> = <v, H u> for L = gR r + gP p (H is a Hessian)."""
    B, N, M, gamma = 3, 5, 6, 0.6
    C, Q = _rand((B, N, M), 21, 2.0), _rand((B, N, M), 22, 2.0, -1.0)
    gr, gp = _rand((B,), 23, 2.0, -1.0), _rand((B,), 24, 2.0, -1.0)
    u = (_rand((B, N, M), 25, 2.0, -1.0), _rand((B, N, M), 26, 2.0, -1.0))
    v = (_rand((B, N, M), 27, 2.0, -1.0), _rand((B, N, M), 28, 2.0, -1.0))
    z = torch.zeros(B, **f64)
    Hu = dp_tangent(C, Q, *u, gr, gp, z, z, gamma)[:2]
    Hv = dp_tangent(C, Q, *v, gr, gp, z, z, gamma)[:2]
    dot = lambda a, b: sum((x * y).sum((1, 2)) for x, y in zip(a, b))
    torch.testing.assert_close(dot(u, Hv), dot(v, Hu), rtol=1e-11, atol=1e-12)
