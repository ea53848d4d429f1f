"""Pins the CPU oracle (``oracle/``) before it is trusted as the GPU checker.

Checks, all on CPU in float64:
* every first-order golden case of the official uDTW / JEANIE code (atol 1e-10);
* the analytic backward against autograd of the differentiable restatement;
* brute-force enumeration over all paths, exact DTW as gamma -> 0, closed forms.
"""

import pytest
import torch

import golden_cases as G
from golden_cases import golden
from oracle import brute, jeanie as OJ, paths as OP, udtw as OU

f64 = dict(dtype=torch.float64)


def close(a, b, tol=1e-10):
    torch.testing.assert_close(a, b, atol=tol, rtol=1e-9)


# ------------------------------------------------------------------ uDTW

def _udtw_autograd(inputs, **kw):
    xs = [x.clone().requires_grad_(True) for x in inputs]
    d, p = OU.udtw(*xs, **kw)
    (d.sum() + 2.0 * p.sum()).backward()
    return [d.detach(), p.detach()] + [x.grad for x in xs]


def _udtw_analytic_one(X, Y, SX, SY, gamma, beta, band, gr, gp):
    """Analytic forward/backward of one d(X,Y) term; returns value, grads."""
    swap = X.shape[1] > Y.shape[1]
    if swap:
        X, Y, SX, SY = Y, X, SY, SX
    vx, vy = SX.squeeze(-1) ** 2, SY.squeeze(-1) ** 2
    r, p, R, P = OU.features_forward(X, Y, vx, vy, gamma, beta, 1e-8, band)
    B = X.shape[0]
    dX, dY, dvx, dvy = OU.features_backward(
        X, Y, vx, vy, R, P, torch.full((B,), gr, **f64), torch.full((B,), gp, **f64),
        gamma, beta, 1e-8)
    dSX = (2.0 * SX.squeeze(-1) * dvx).unsqueeze(-1)
    dSY = (2.0 * SY.squeeze(-1) * dvy).unsqueeze(-1)
    if swap:
        dX, dY, dSX, dSY = dY, dX, dSY, dSX
    return r, p, [dX, dY, dSX, dSY]


def _udtw_analytic(inputs, gamma, beta=0.7, normalize=False, bandwidth=None):
    X, Y, SX, SY = inputs
    band = bandwidth or 0.0
    r, p, g = _udtw_analytic_one(X, Y, SX, SY, gamma, beta, band, 1.0, 2.0)
    if not normalize:
        return [r, p] + g
    rx, px, gx = _udtw_analytic_one(X, X, SX, SX, gamma, beta, band, -0.5, -1.0)
    ry, py, gy = _udtw_analytic_one(Y, Y, SY, SY, gamma, beta, band, -0.5, -1.0)
    grads = [g[0] + gx[0] + gx[1], g[1] + gy[0] + gy[1],
             g[2] + gx[2] + gx[3], g[3] + gy[2] + gy[3]]
    return [r - 0.5 * (rx + ry), p - 0.5 * (px + py)] + grads


@pytest.mark.parametrize("N,M", G.UDTW_SHAPES)
@pytest.mark.parametrize("gamma", G.GAMMAS)
@pytest.mark.parametrize("normalize", [False, True])
def test_udtw_matches_golden(N, M, gamma, normalize):
    ref = golden("udtw.matches", N=N, M=M, gamma=gamma, normalize=normalize)
    for got in (_udtw_autograd(ref["inputs"], gamma=gamma, beta=0.7, normalize=normalize),
                _udtw_analytic(ref["inputs"], gamma, normalize=normalize)):
        for a, b in zip(got, ref["outputs"]):
            close(a, b)


@pytest.mark.parametrize("N,M,bandwidth", G.UDTW_BANDS)
def test_udtw_band_golden(N, M, bandwidth):
    ref = golden("udtw.bandwidth", N=N, M=M, bandwidth=bandwidth)
    for got in (_udtw_autograd(ref["inputs"], gamma=0.1, beta=0.7, bandwidth=bandwidth),
                _udtw_analytic(ref["inputs"], 0.1, bandwidth=bandwidth)):
        for a, b in zip(got, ref["outputs"]):
            close(a, b)


@pytest.mark.parametrize("beta", G.UDTW_BETAS)
def test_udtw_beta_golden(beta):
    ref = golden("udtw.beta", beta=beta)
    for got in (_udtw_autograd(ref["inputs"], gamma=0.1, beta=beta),
                _udtw_analytic(ref["inputs"], 0.1, beta=beta)):
        for a, b in zip(got, ref["outputs"]):
            close(a, b)


@pytest.mark.parametrize("case", ["udtw.large", "udtw.float32"])
def test_udtw_larger_golden(case):
    ref = golden(case, B=2, N=40, M=50) if case == "udtw.large" else golden(case)
    got = _udtw_analytic(ref["inputs"], 0.1)
    for a, b in zip(got, ref["outputs"]):
        close(a, b)


def test_pairwise_matrices_golden():
    ref = golden("udtw.pairwise_matrices")
    X, Y, SX, SY = ref["inputs"]
    cost, pen, sq_raw, var_raw = OU.pairwise(X, Y, SX.squeeze(-1) ** 2, SY.squeeze(-1) ** 2,
                                             0.5, 1e-8)
    want = ref["outputs"]
    torch.testing.assert_close(cost, want[0], atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(pen, want[1], atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(var_raw.clamp_min(1e-8), want[2], atol=1e-12, rtol=1e-10)


def test_udtw_brute_force():
    g = torch.Generator().manual_seed(11)
    for N, M in [(1, 1), (1, 4), (3, 4), (4, 4), (4, 2)]:
        C = torch.rand(1, N, M, generator=g, **f64)
        Q = torch.randn(1, N, M, generator=g, **f64)
        for gamma in (0.05, 1.0):
            r, p, _, _ = OU.dp_forward(C, Q, gamma)
            rb, pb = brute.udtw_value(C[0], Q[0], gamma)
            close(r[0], rb)
            close(p[0], pb)


def test_udtw_analytic_backward_matches_autograd():
    g = torch.Generator().manual_seed(3)
    for N, M, band in [(5, 7, 0.0), (7, 5, 0.0), (8, 8, 2.0), (1, 6, 0.0)]:
        C = torch.rand(2, N, M, generator=g, **f64)
        Q = torch.randn(2, N, M, generator=g, **f64)
        gr, gp = torch.randn(2, generator=g, **f64), torch.randn(2, generator=g, **f64)
        r, p, R, P = OU.dp_forward(C, Q, 0.3, band)
        dC, dQ = OU.dp_backward(C, Q, R, P, gr, gp, 0.3)
        c, q = C.clone().requires_grad_(), Q.clone().requires_grad_()
        rv, pv = OU.dp_value(c, q, 0.3, band)
        close(rv, r)
        close(pv, p)
        ac, aq = torch.autograd.grad((gr * rv).sum() + (gp * pv).sum(), (c, q))
        close(dC, ac)
        close(dQ, aq)


def test_unreachable_band_gives_inf():
    C = torch.rand(1, 3, 9, **f64)
    r, p, R, P = OU.dp_forward(C, torch.zeros_like(C), 0.1, 2.0)
    assert torch.isinf(r).all() and (p == 0).all()


# ------------------------------------------------------------ JEANIE / FVM

def _value_and_grad(fn, x):
    x = x.clone().requires_grad_(True)
    out = fn(x)
    (g,) = torch.autograd.grad(out.sum(), x)
    return out.detach(), g


def _jeanie_analytic(cost5, s1, s2, gamma, grad_R=None):
    """Analytic (out, R, dC) with the T <= U transposition of the reference."""
    tr = cost5.shape[3] > cost5.shape[4]
    c = cost5.transpose(3, 4) if tr else cost5
    out, R = OJ.forward(c, s1, s2, gamma)
    gR = None if grad_R is None else (grad_R.transpose(3, 4) if tr else grad_R)
    dC = OJ.backward(c, R, torch.ones_like(out), s1, s2, gamma, gR)
    if tr:
        R, dC = R.transpose(3, 4), dC.transpose(3, 4)
    return out, R, dC


@pytest.mark.parametrize("T,U", G.SDTW_SHAPES)
@pytest.mark.parametrize("gamma", G.GAMMAS)
def test_soft_dtw_golden(T, U, gamma):
    ref = golden("jeanie.soft_dtw", T=T, U=U, gamma=gamma)
    v, g = _value_and_grad(lambda c: OJ.soft_dtw_from_cost(c[None], gamma=gamma)[0], ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])
    out, _, dC = _jeanie_analytic(ref["cost"][None, None, None], 0, 0, gamma)
    close(out[0], ref["value"])
    close(dC[0, 0, 0], ref["grad"])


@pytest.mark.parametrize("K,T,U", G.JEANIE_1D_SHAPES)
@pytest.mark.parametrize("shift", G.JEANIE_1D_SHIFTS)
def test_jeanie_1d_golden(K, T, U, shift):
    ref = golden("jeanie.jeanie_1d", K=K, T=T, U=U, shift=shift)
    v, g = _value_and_grad(
        lambda c: OJ.jeanie_from_cost(c[None], gamma=0.1, max_shift=shift)[0], ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])
    s1, _ = OJ.clamp_shifts(K, 1, shift, 0)
    out, R, dC = _jeanie_analytic(ref["cost"][None, :, None], s1, 0, 0.1)
    close(out[0], ref["value"])
    close(dC[0, :, 0], ref["grad"])
    close(R[0, :, 0], ref["accumulator"])


@pytest.mark.parametrize("K1,K2,T,U", G.JEANIE_2D_SHAPES)
@pytest.mark.parametrize("s_az,s_alt", G.JEANIE_2D_SHIFTS)
def test_jeanie_2d_golden(K1, K2, T, U, s_az, s_alt):
    ref = golden("jeanie.jeanie_2d", K1=K1, K2=K2, T=T, U=U, s_az=s_az, s_alt=s_alt)
    v, g = _value_and_grad(
        lambda c: OJ.jeanie_from_cost(c[None], gamma=0.1, max_shift=(s_az, s_alt))[0],
        ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])
    s1, s2 = OJ.clamp_shifts(K1, K2, s_az, s_alt)
    out, _, dC = _jeanie_analytic(ref["cost"][None], s1, s2, 0.1)
    close(out[0], ref["value"])
    close(dC[0], ref["grad"])


def test_jeanie_batched_golden():
    ref = golden("jeanie.batched")
    close(OJ.jeanie_from_cost(ref["cost_1d"], gamma=0.1, max_shift=1), ref["value_1d"])
    close(OJ.jeanie_from_cost(ref["cost_2d"], gamma=0.1, max_shift=(1, 1)), ref["value_2d"])


@pytest.mark.parametrize("name,shape", G.FVM_CASES)
def test_fvm_golden(name, shape):
    ref = golden("jeanie.fvm", name=name)
    v, g = _value_and_grad(lambda c: OJ.fvm_from_cost(c[None], gamma=0.1)[0], ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])
    close(OJ.fvm_backward(ref["cost"][None], torch.ones(1, **f64), 0.1)[0], ref["grad"])
    close(OJ.fvm_from_cost(ref["batch"], gamma=0.1), ref["batch_value"])


@pytest.mark.parametrize("name,shape,shift", G.LARGE_COST)
def test_large_golden(name, shape, shift):
    ref = golden("jeanie.large", name=name, shape=shape)
    cost = ref["cost"]
    if name == "soft_dtw":
        c5, s1, s2 = cost[None, None, None], 0, 0
        v = OJ.soft_dtw_from_cost(cost[None], gamma=0.1)[0]
        close(v, ref["value"])
    elif name.startswith("fvm"):
        v = OJ.fvm_from_cost(cost[None], gamma=0.1)[0]
        close(v, ref["value"])
        close(OJ.fvm_backward(cost[None], torch.ones(1, **f64), 0.1)[0], ref["grad"])
        return
    elif name == "jeanie_1d_from_cost":
        c5, s1, s2 = cost[None, :, None], min(shift, cost.shape[0] - 1), 0
    else:
        c5 = cost[None]
        s1, s2 = OJ.clamp_shifts(cost.shape[0], cost.shape[1], *shift)
    out, _, dC = _jeanie_analytic(c5, s1, s2, 0.1)
    close(out[0], ref["value"])
    close(dC.reshape(cost.shape), ref["grad"])


def test_softmin_golden():
    ref = golden("jeanie.softmin")
    v = ref["v"]
    torch.testing.assert_close(-0.3 * torch.logsumexp(-v / 0.3, dim=1), ref["outputs"][0])
    torch.testing.assert_close(-0.3 * torch.logsumexp(-v.reshape(-1) / 0.3, dim=0),
                               ref["outputs"][1])


@pytest.mark.parametrize("name", G.DISTANCES)
def test_distances_golden(name):
    ref = golden("jeanie.distance", name=name)
    fn = getattr(OJ, name)
    q, s = ref["q"].clone().requires_grad_(), ref["s"].clone().requires_grad_()
    out = fn(q, s)
    close(out, ref["value"])
    for a, b in zip(torch.autograd.grad(out.sum(), (q, s)), ref["grads"]):
        close(a, b)
    close(fn(ref["qb"], ref["sb"]), ref["batch_value"])


def test_end_to_end_golden():
    ref = golden("jeanie.end_to_end")
    q, s = ref["q"].clone().requires_grad_(), ref["s"].clone().requires_grad_()
    d = OJ.jeanie_from_cost(OJ.euclidean_cost(q[None], s[None]), gamma=0.1, max_shift=1)[0]
    close(d, ref["value"])
    for a, b in zip(torch.autograd.grad(d, (q, s)), ref["grads"]):
        close(a, b)


_COST = {"euclidean": OJ.euclidean_cost, "sqeuclidean": OJ.squared_euclidean_cost,
         "rbf": OJ.rbf_cost}


@pytest.mark.parametrize("metric", G.METRICS)
@pytest.mark.parametrize("K,T,U,shift", G.FEATURES_1D)
def test_features_1d_golden(metric, K, T, U, shift):
    ref = golden("jeanie.features_1d", metric=metric, K=K, T=T, U=U, shift=shift)
    q, s = ref["q"].clone().requires_grad_(), ref["s"].clone().requires_grad_()
    d = OJ.jeanie_from_cost(_COST[metric](q, s), gamma=0.1, max_shift=shift)
    close(d, ref["value"])
    for a, b in zip(torch.autograd.grad(d.sum(), (q, s)), ref["grads"]):
        close(a, b)


@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean"])
def test_features_2d_golden(metric):
    ref = golden("jeanie.features_2d", metric=metric)
    q, s = ref["q"].clone().requires_grad_(), ref["s"].clone().requires_grad_()
    B, K1, K2, T, D = q.shape
    cost = _COST[metric](q.reshape(B, K1 * K2, T, D), s).reshape(B, K1, K2, T, -1)
    d, acc = OJ.jeanie_from_cost(cost, gamma=0.1, max_shift=(1, 1), return_accumulator=True)
    close(d, ref["value"])
    for a, b in zip(torch.autograd.grad(d.sum(), (q, s)), ref["grads"]):
        close(a, b)
    close(acc[0].detach(), ref["accumulator"])


@pytest.mark.parametrize("K,T,U,shift", G.ACCUMULATOR_COST)
def test_accumulator_seed_golden(K, T, U, shift):
    """The dL/dR seed of the analytic backward reproduces the official gradient."""
    ref = golden("parity.accumulator_cost", K=K, T=T, U=U, shift=shift)
    cost = ref["cost"][None, :, None]
    s1 = min(shift, K - 1)
    tr = T > U
    c = cost.transpose(3, 4) if tr else cost
    out, R = OJ.forward(c, s1, 0, 0.3)
    gR = 0.1 * 2.0 * R / R.numel()
    dC = OJ.backward(c, R, torch.ones_like(out), s1, 0, 0.3, gR)
    if tr:
        dC = dC.transpose(3, 4)
    close(dC[0, :, 0], ref["grad"])


def test_accumulator_2d_golden():
    ref = golden("parity.accumulator_2d")
    c = ref["cost"][None]
    out, R = OJ.forward(c, 1, 1, 0.3)
    dC = OJ.backward(c, R, torch.ones_like(out), 1, 1, 0.3, torch.cos(R))
    close(dC[0], ref["grad"])


@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean"])
def test_accumulator_features_golden(metric):
    ref = golden("parity.accumulator_features", metric=metric)
    q, s = ref["q"].clone().requires_grad_(), ref["s"].clone().requires_grad_()
    d, R = OJ.jeanie_from_cost(_COST[metric](q[None], s[None]), gamma=0.3, max_shift=1,
                               return_accumulator=True)
    loss = d[0] + 0.1 * (R ** 2).mean()
    for a, b in zip(torch.autograd.grad(loss, (q, s)), ref["grads"]):
        close(a, b)


@pytest.mark.parametrize("gamma", [0.1, 1.0])
@pytest.mark.parametrize("K,T,U,shift", [(3, 4, 5, 1), (3, 3, 4, 2), (1, 4, 4, 0), (2, 1, 5, 1)])
def test_jeanie_brute_force(gamma, K, T, U, shift):
    g = torch.Generator().manual_seed(K * 100 + T * 10 + U)
    cost = torch.rand(K, T, U, generator=g, **f64)
    value, pm, paths, w = brute.soft_value_and_grad(cost, gamma, shift)
    out, _, dC = _jeanie_analytic(cost[None, :, None], min(shift, K - 1), 0, gamma)
    close(out[0], value)
    close(dC[0, :, 0], pm, tol=1e-9)
    hard = OP.optimal_path(cost[None].numpy(), max_shift=shift)[0]
    assert hard == paths[int(w.argmin())]


def test_soft_dtw_gamma_to_zero_is_dtw():
    g = torch.Generator().manual_seed(5)
    cost = torch.rand(1, 9, 12, generator=g, **f64)
    v = OJ.soft_dtw_from_cost(cost, gamma=1e-4)[0]
    assert abs(float(v) - brute.exact_dtw(cost[0])) < 1e-2
    path = OP.optimal_path(cost.numpy())[0]
    assert abs(sum(float(cost[0, t, u]) for t, u in path) - brute.exact_dtw(cost[0])) < 1e-12


def test_closed_forms():
    g = torch.Generator().manual_seed(8)
    c = torch.rand(2, 1, 1, 1, 7, generator=g, **f64)   # a single row: one path
    out, R, dC = _jeanie_analytic(c, 0, 0, 0.5)
    close(out, c.sum((1, 2, 3, 4)))
    close(dC, torch.ones_like(c))
    c1 = torch.rand(3, 1, 1, 1, 1, generator=g, **f64)
    out, _, dC = _jeanie_analytic(c1, 0, 0, 0.5)
    close(out, c1.flatten())
    # K = 1 JEANIE equals soft-DTW; one viewpoint axis equals K2 = 1
    c = torch.rand(2, 1, 1, 6, 8, generator=g, **f64)
    close(OJ.forward(c, 0, 0, 0.2)[0], OU.dp_forward(c[:, 0, 0], torch.zeros_like(c[:, 0, 0]),
                                                     0.2)[0])
