"""The reference-named operators (``torchwarp_udtw::*``, ``torchwarp_jeanie::*``)
on the GPU: each forward / backward pair called by name, as code written for
the reference's operators calls them, gives the public API's values and
gradients (which the other GPU tests hold against the oracle and the golden
data); ``torch.library.opcheck`` checks schema and fake implementations."""

import pytest
import torch

import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

f64 = torch.float64
U_, J_ = torch.ops.torchwarp_udtw, torch.ops.torchwarp_jeanie


def _rand(shape, seed, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return (shift + scale * torch.rand(shape, generator=g, dtype=f64)).cuda()


def _close(a, b, tol=1e-10):
    den = b.abs().max().item()
    return (a - b).abs().max().item() <= tol * (den if den > 0 else 1.0)


@pytest.mark.parametrize("band", [0.0, 6.0])
def test_udtw_dp_pair_by_name(band):
    B, N, M, gamma = 3, 30, 34, 0.5
    C, Q = _rand((B, N, M), 1, 3.0), _rand((B, N, M), 2, 0.5)
    gr, gp = _rand((B,), 3, 1.0, 0.5), _rand((B,), 4, 1.0, 0.5)
    out_r, out_p, R, P = U_.dp(C, Q, gamma, band, "auto")
    dC, dQ = U_.dp_backward(C, Q, R, P, gr, gp, gamma, band, "auto")
    c, q = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    d, p = TF.udtw_from_cost(c, q, gamma=gamma, bandwidth=band or None)
    (d * gr + p * gp).sum().backward()
    assert _close(out_r, d.detach()) and _close(out_p, p.detach())
    assert _close(dC, c.grad) and _close(dQ, q.grad)


@pytest.mark.parametrize("D", [1, 3])
def test_udtw_fused_pair_by_name(D):
    """vx, vy are variances, as the reference's op takes them."""
    B, N, M, gamma, beta, eps = 2, 20, 23, 0.7, 0.8, 1e-8
    X, Y = _rand((B, N, D), 5, 2.0, -1.0), _rand((B, M, D), 6, 2.0, -1.0)
    sx, sy = _rand((B, N, 1), 7, 1.0, 0.5), _rand((B, M, 1), 8, 1.0, 0.5)
    gr, gp = _rand((B,), 9, 1.0, 0.5), _rand((B,), 10, 1.0, 0.5)
    vx, vy = sx[..., 0] ** 2, sy[..., 0] ** 2
    f = U_.fused(X, Y, vx, vy, gamma, beta, eps, 0.0, "auto")
    assert len(f) == 7
    dX, dY, dvx, dvy = U_.fused_backward(X, Y, vx, vy, f[2], f[3], f[4], f[5], f[6], gr, gp,
                                         gamma, beta, eps, 0.0, "auto")
    xs = [t.clone().requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = TF.udtw(*xs, beta=beta, gamma=gamma, eps=eps)
    (d * gr + p * gp).sum().backward()
    assert _close(f[0], d.detach()) and _close(f[1], p.detach())
    assert _close(dX, xs[0].grad) and _close(dY, xs[1].grad)
    # d/dsigma = d/dvar * 2 sigma
    assert _close(dvx * 2 * sx[..., 0], xs[2].grad[..., 0])
    assert _close(dvy * 2 * sy[..., 0], xs[3].grad[..., 0])


def test_jeanie_dp_pair_by_name():
    B, K1, K2, T, U, gamma = 4, 3, 2, 9, 8, 0.3
    cost = _rand((B, K1, K2, T, U), 11, 2.0)
    g_out, g_R = _rand((B,), 12, 1.0, 0.5), _rand((B, K1, K2, T, U), 13, 1.0, -0.5)
    out, R_d, R = J_.dp(cost, 1, 1, gamma, "auto", True)
    d = J_.dp_backward(cost, R_d, g_out, g_R, 1, 1, gamma, "auto")
    c = cost.clone().requires_grad_(True)
    o2, R2 = TF.jeanie_from_cost(c, gamma=gamma, max_shift=1, return_accumulator=True)
    ((o2 * g_out).sum() + (R2 * g_R).sum()).backward()
    assert _close(out, o2.detach()) and _close(R, R2.detach()) and _close(d, c.grad)
    # without the accumulator: the R output is empty and grad_R may be None
    out3, R_d3, R3 = J_.dp(cost, 1, 1, gamma, "auto", False)
    assert R3.numel() == 0 and _close(out3, out)
    d3 = J_.dp_backward(cost, R_d3, g_out, None, 1, 1, gamma, "auto")
    c2 = cost.clone().requires_grad_(True)
    (TF.jeanie_from_cost(c2, gamma=gamma, max_shift=1) * g_out).sum().backward()
    assert _close(d3, c2.grad)


@pytest.mark.parametrize("metric", [0, 1], ids=["sqeuclidean", "euclidean"])
def test_jeanie_features_pair_by_name(metric):
    B, K1, K2, T, U, D, gamma = 3, 3, 1, 7, 6, 5, 0.2
    q, s = _rand((B, K1, K2, T, D), 14, 2.0, -1.0), _rand((B, U, D), 15, 2.0, -1.0)
    g_out = _rand((B,), 16, 1.0, 0.5)
    fo = J_.features(q, s, 1, 0, gamma, metric, "auto", False)
    assert len(fo) == 6
    dq, ds = J_.features_backward(q, s, fo[1], fo[3], fo[4], fo[5], g_out, None, 1, 0, gamma,
                                  metric, "auto")
    qq, ss = q.clone().requires_grad_(True), s.clone().requires_grad_(True)
    o = TF.jeanie(qq, ss, gamma=gamma, max_shift=(1, 0),
                  metric="euclidean" if metric else "sqeuclidean")
    (o * g_out).sum().backward()
    assert _close(fo[0], o.detach()) and _close(dq, qq.grad) and _close(ds, ss.grad)


def test_opcheck_schema_and_fake():
    C, Q = _rand((2, 6, 7), 17), _rand((2, 6, 7), 18)
    tests = ("test_schema", "test_faketensor")
    torch.library.opcheck(U_.dp.default, (C, Q, 1.0, 0.0, "auto"), test_utils=tests)
    out = U_.dp(C, Q, 1.0, 0.0, "auto")
    torch.library.opcheck(U_.dp_backward.default, (C, Q, out[2], out[3], out[0], out[1], 1.0, 0.0,
                                                   "auto"), test_utils=tests)
    cj = _rand((2, 3, 1, 5, 4), 19)
    torch.library.opcheck(J_.dp.default, (cj, 1, 0, 0.1, "auto", True), test_utils=tests)
