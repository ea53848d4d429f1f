"""The autograd contract on the HIP path against the reference's stored values.

The reference's parity suites (tests/test_udtw_parity.py:48-137,
tests/test_jeanie_parity.py:54-230) check higher-order gradients
(create_graph / MAML, a third derivative), forward mode, every torch.func
transform and vmap against outputs of the official pure-autograd code, kept
in tests/golden. These run the same losses through torchwarp_amd on the GPU
in float64: first-order reverse goes through the HIP backward kernels, the
higher orders and jvp through the ops' registered rules.
"""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF
from torchwarp_amd.jeanie.functional import _jeanie_dp, _jeanie_dp_features

import golden_cases as G
from golden_cases import golden

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"
METHODS = ["gemm", "diff"]


def _close(a, b, tol=1e-9):
    torch.testing.assert_close(a.detach().cpu(), b, atol=tol, rtol=tol)


def _scalar(module):
    def f(X, Y, SX, SY):
        d, p = module(X, Y, SX, SY)
        return d.sum() + 2.0 * p.sum()
    return f


# ------------------------------------------------------------------- uDTW

@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("normalize,bandwidth", G.UDTW_MAML)
def test_udtw_maml_meta_gradient(method, normalize, bandwidth):
    ref = golden("udtw.maml", normalize=normalize, bandwidth=bandwidth)
    X, Y, SX, SY = (t.to(DEV) for t in ref["inputs"])
    f = _scalar(tw.UDTW(gamma=0.3, beta=0.8, normalize=normalize, bandwidth=bandwidth,
                        method=method))
    w = ref["W0"].to(DEV).requires_grad_()
    g, = torch.autograd.grad(f(X @ w.T, Y @ w.T, SX, SY), w, create_graph=True)
    w2 = w - 0.1 * g
    _close(torch.autograd.grad(f(X @ w2.T, Y @ w2.T, SX, SY), w)[0], ref["meta_grad"])


@pytest.mark.parametrize("method", METHODS)
def test_udtw_third_derivative(method):
    ref = golden("udtw.third_derivative")
    X, Y, SX, SY = (t.to(DEV) for t in ref["inputs"])
    V = ref["V"].to(DEV)
    f = _scalar(tw.UDTW(gamma=0.5, beta=0.8, method=method))
    t = torch.zeros((), device=DEV, dtype=torch.float64).requires_grad_()
    y = f(X + t * V, Y, SX, SY)
    for _ in range(3):
        y, = torch.autograd.grad(y, t, create_graph=True)
    _close(y, ref["d3"], tol=1e-7)


@pytest.mark.parametrize("method", METHODS)
def test_udtw_torch_func_transforms(method):
    ref = golden("udtw.func")
    X, Y, SX, SY = (t.to(DEV) for t in ref["inputs"])
    f = lambda x: _scalar(tw.UDTW(gamma=0.4, beta=0.8, method=method))(x, Y, SX, SY)
    J = ref["jacobian"]
    _close(torch.func.grad(f)(X), J)
    _close(torch.func.jacrev(f)(X), J)
    _close(torch.func.jacfwd(f)(X), J)
    _, jvp = torch.func.jvp(f, (X,), (ref["v"].to(DEV),))
    _close(jvp, ref["jvp"])
    H = ref["hessian"]
    _close(torch.func.hessian(f)(X), H, tol=1e-7)
    _close(torch.func.jacrev(torch.func.jacrev(f))(X), H, tol=1e-7)


@pytest.mark.parametrize("method", METHODS)
def test_udtw_vmap(method):
    ref = golden("udtw.vmap")
    X, Y, SX, SY = (t.to(DEV) for t in ref["inputs"])
    stack = lambda t: torch.stack([t, 1.1 * t, 0.9 * t])
    m = tw.UDTW(gamma=0.3, beta=0.5, method=method)
    d, p = torch.func.vmap(m)(stack(X), stack(Y), stack(SX), stack(SY))
    _close(d, ref["distance"])
    _close(p, ref["penalty"])
    per = torch.func.vmap(torch.func.grad(
        lambda x, y, sx, sy: _scalar(m)(x[None], y[None], sx[None], sy[None])))(X, Y, SX, SY)
    full = torch.func.grad(_scalar(m))(X, Y, SX, SY)
    torch.testing.assert_close(per, full, atol=1e-9, rtol=1e-9)


def test_udtw_gradgradcheck():
    kw = dict(device=DEV, dtype=torch.float64)
    g = torch.Generator().manual_seed(12)
    cost = torch.rand(2, 3, 4, generator=g, dtype=torch.float64).to(DEV).requires_grad_()
    pen = torch.randn(2, 3, 4, generator=g, dtype=torch.float64).to(DEV).requires_grad_()
    assert torch.autograd.gradgradcheck(lambda c, p: TF.udtw_from_cost(c, p, gamma=0.4),
                                        (cost, pen))
    X, Y = (torch.rand(1, L, 2, **kw).requires_grad_() for L in (3, 4))
    SX, SY = ((0.5 + torch.rand(1, L, 1, **kw)).requires_grad_() for L in (3, 4))
    assert torch.autograd.gradgradcheck(lambda *a: TF.udtw(*a, beta=0.7, gamma=0.4),
                                        (X, Y, SX, SY))


# ---------------------------------------------------------------- JEANIE

def _cost_loss(cost, shift):
    d, R = TF.jeanie_from_cost(cost[None], gamma=0.3, max_shift=shift, return_accumulator=True)
    return d[0] + 0.1 * (R ** 2).mean()


def _feat_loss(q, s, metric, shift=1):
    d, R = TF.jeanie(q[None], s[None], gamma=0.3, max_shift=shift, metric=metric,
                     return_accumulator=True)
    return d[0] + 0.1 * (R ** 2).mean()


@pytest.mark.parametrize("path", ["cost", "euclidean", "sqeuclidean"])
def test_jeanie_maml_meta_gradient(path):
    ref = golden("parity.maml", path=path)

    def loss(qw, sw):
        if path == "cost":
            return _cost_loss(tw.euclidean_cost(qw[None], sw[None])[0], 1)
        return _feat_loss(qw, sw, path)

    w = ref["W0"].to(DEV).requires_grad_()
    a, b = ref["q"].to(DEV), ref["s"].to(DEV)
    g, = torch.autograd.grad(loss(a @ w.T, b @ w.T), w, create_graph=True)
    w2 = w - 0.1 * g
    _close(torch.autograd.grad(loss(a @ w2.T, b @ w2.T), w)[0], ref["meta_grad"])


def _second_order_fn(method, s):
    if method == "jeanie_cost":
        return lambda x: TF.jeanie_from_cost(x[None], gamma=0.3, max_shift=1)[0]
    if method == "jeanie_features":
        return lambda x: TF.jeanie(x[None], s[None], gamma=0.3, max_shift=1)[0]
    if method == "fvm":
        return lambda x: TF.fvm_from_cost(x[None], gamma=0.3)[0]
    return lambda x: TF.soft_dtw_from_cost(x[None], gamma=0.3)[0]


@pytest.mark.parametrize("method", G.SECOND_ORDER)
def test_second_order_without_accumulator(method):
    ref = golden("parity.second_order", method=method)
    f = _second_order_fn(method, ref["s"].to(DEV))
    x = ref["x"].to(DEV)
    J = ref["jacobian"]
    _close(torch.func.grad(f)(x), J)
    _close(torch.func.jacrev(f)(x), J)
    _close(torch.func.jacfwd(f)(x), J)
    _, jvp = torch.func.jvp(f, (x,), (ref["v"].to(DEV),))
    _close(jvp, ref["jvp"])
    H = ref["hessian"]
    _close(torch.func.hessian(f)(x), H, tol=1e-7)
    _close(torch.func.jacrev(torch.func.jacrev(f))(x), H, tol=1e-7)
    _close(torch.autograd.functional.hessian(f, x), H, tol=1e-7)


@pytest.mark.parametrize("method", G.SECOND_ORDER)
def test_maml_without_accumulator(method):
    ref = golden("parity.maml_without_accumulator", method=method)

    def loss(a, b):
        if method == "jeanie_cost":
            return TF.jeanie_from_cost(tw.euclidean_cost(a[None], b[None]), gamma=0.3,
                                       max_shift=1)[0]
        if method == "jeanie_features":
            return TF.jeanie(a[None], b[None], gamma=0.3, max_shift=1)[0]
        if method == "fvm":
            return TF.fvm(a[None], b[None], gamma=0.3)[0]
        cost = ((a[:, None] - b[None]) ** 2).sum(-1)
        return TF.soft_dtw_from_cost(cost[None], gamma=0.3)[0]

    w = ref["W0"].to(DEV).requires_grad_()
    a, b = ref["q"].to(DEV), ref["s"].to(DEV)
    g, = torch.autograd.grad(loss(a @ w.T, b @ w.T), w, create_graph=True)
    w2 = w - 0.1 * g
    _close(torch.autograd.grad(loss(a @ w2.T, b @ w2.T), w)[0], ref["meta_grad"])


@pytest.mark.parametrize("path", ["cost", "euclidean"])
def test_jeanie_torch_func_transforms(path):
    ref = golden("parity.func", path=path)
    if path == "cost":
        f = lambda c: _cost_loss(c, 1)
    else:
        s = ref["s"].to(DEV)
        f = lambda qq: _feat_loss(qq, s, path)
    x = ref["x"].to(DEV)
    J = ref["jacobian"]
    _close(torch.func.grad(f)(x), J)
    _close(torch.func.jacrev(f)(x), J)
    _close(torch.func.jacfwd(f)(x), J)
    _, jvp = torch.func.jvp(f, (x,), (ref["v"].to(DEV),))
    _close(jvp, ref["jvp"])
    H = ref["hessian"]
    _close(torch.func.hessian(f)(x), H, tol=1e-7)
    _close(torch.func.jacrev(torch.func.jacrev(f))(x), H, tol=1e-7)


def test_jeanie_vmap():
    ref = golden("parity.vmap")
    got = torch.func.vmap(lambda c: TF.jeanie_from_cost(c, gamma=0.3, max_shift=1))(
        ref["cost"].to(DEV))
    _close(got, ref["cost_value"])
    q, s = ref["q"].to(DEV), ref["s"].to(DEV)
    got = torch.func.vmap(lambda a, b: TF.jeanie(a, b, gamma=0.3, max_shift=1))(q, s)
    _close(got, ref["features_value"])
    f = lambda a, b: TF.jeanie(a, b, gamma=0.3, max_shift=1)
    per = torch.func.vmap(torch.func.grad(lambda a, b: f(a[None], b[None])[0]))(q[0], s[0])
    full = torch.func.grad(lambda a, b: f(a, b).sum())(q[0], s[0])
    torch.testing.assert_close(per, full, atol=1e-9, rtol=1e-9)


def test_jeanie_gradgradcheck():
    kw = dict(device=DEV, dtype=torch.float64)
    cost = torch.rand(2, 2, 2, 3, 4, **kw).requires_grad_()
    f = lambda c: tuple(_jeanie_dp(c, 0.5, 1, 1, "auto", return_accumulator=True))
    assert torch.autograd.gradgradcheck(f, (cost,))
    q = torch.randn(1, 2, 1, 3, 2, **kw).requires_grad_()
    s = torch.randn(1, 4, 2, **kw).requires_grad_()
    for metric in ("euclidean", "sqeuclidean"):
        g = lambda q, s: tuple(_jeanie_dp_features(q, s, 0.5, 1, 0, metric, "auto",
                                                   return_accumulator=True))
        assert torch.autograd.gradgradcheck(g, (q, s))
    c2 = torch.rand(2, 3, 3, 4, **kw).requires_grad_()
    assert torch.autograd.gradgradcheck(lambda c: TF.jeanie_from_cost(c, gamma=0.5, max_shift=1),
                                        (c2,))
    assert torch.autograd.gradgradcheck(lambda c: TF.fvm_from_cost(c, gamma=0.5), (c2,))
    assert torch.autograd.gradgradcheck(lambda c: TF.soft_dtw_from_cost(c[:, 0], gamma=0.5),
                                        (c2,))
    q2 = torch.randn(1, 2, 3, 2, **kw).requires_grad_()
    for metric in ("euclidean", "sqeuclidean", "rbf"):
        assert torch.autograd.gradgradcheck(
            lambda q, s: TF.jeanie(q, s, gamma=0.5, max_shift=1, metric=metric), (q2, s))
        assert torch.autograd.gradgradcheck(
            lambda q, s: TF.fvm(q, s, gamma=0.5, metric=metric), (q2, s))


@pytest.mark.parametrize("name", ["udtw.softmin", "jeanie.softmin"])
def test_softmin_helpers(name):
    """softmin / softmin_weights (sdtw.py) on device tensors, as the reference's
    tests/test_udtw.py:95-100 and tests/test_jeanie.py:121-124 check them."""
    ref = golden(name)
    v, want = ref["v"].to(DEV), ref["outputs"]
    _close(TF.softmin(v, 0.3, dim=1), want[0])
    _close(TF.softmin(v, 0.3), want[1])
    if len(want) > 2:
        _close(TF.softmin_weights(v, 0.3, dim=1), want[2])


# ------------------------------------------------- torch.compile and autocast
# (reference tests/test_udtw_parity.py:142-172, tests/test_jeanie_parity.py:246-284)

def _udtw_inputs(B=3, N=5, M=7, D=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(B, N, D, generator=g, dtype=torch.float64),
            torch.rand(B, M, D, generator=g, dtype=torch.float64),
            0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64),
            0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64))


@pytest.mark.parametrize("method", METHODS)
def test_udtw_torch_compile_fullgraph(method):
    torch._dynamo.reset()
    X, Y, SX, SY = (t.to(DEV).requires_grad_() for t in _udtw_inputs())
    f = _scalar(tw.UDTW(gamma=0.3, beta=0.8, normalize=True, method=method))
    compiled = torch.compile(f, fullgraph=True)
    want = f(X, Y, SX, SY)
    got = compiled(X, Y, SX, SY)
    _close(got, want.detach().cpu())
    for a, b in zip(torch.autograd.grad(got, (X, Y, SX, SY)),
                    torch.autograd.grad(want, (X, Y, SX, SY))):
        _close(a, b.detach().cpu())


@pytest.mark.parametrize("path", ["cost", "euclidean"])
def test_jeanie_torch_compile_fullgraph(path):
    torch._dynamo.reset()
    q = torch.randn(2, 3, 5, 4, device=DEV, dtype=torch.float64).requires_grad_()
    s = torch.randn(2, 6, 4, device=DEV, dtype=torch.float64).requires_grad_()

    def f(q, s):
        if path == "cost":
            d, R = TF.jeanie_from_cost(tw.euclidean_cost(q, s), gamma=0.3, max_shift=1,
                                       return_accumulator=True)
        else:
            d, R = TF.jeanie(q, s, gamma=0.3, max_shift=1, return_accumulator=True)
        return d.sum() + 0.1 * (R ** 2).mean()

    compiled = torch.compile(f, fullgraph=True)
    want, got = f(q, s), compiled(q, s)
    _close(got, want.detach().cpu())
    for a, b in zip(torch.autograd.grad(got, (q, s)), torch.autograd.grad(want, (q, s))):
        _close(a, b.detach().cpu())


def test_autocast_runs_in_float32():
    X, Y, SX, SY = (t.float().to(DEV).requires_grad_() for t in _udtw_inputs(B=2, N=5, M=6))
    lin = torch.nn.Linear(4, 4).to(DEV)
    for method in METHODS:
        m = tw.UDTW(gamma=0.3, method=method)
        with torch.autocast("cuda", dtype=torch.float16):
            d, p = m(lin(X), lin(Y), SX, SY)
        assert d.dtype == torch.float32 and p.dtype == torch.float32
        (d.sum() + p.sum()).backward()
        assert torch.isfinite(X.grad).all()
        ref_d, _ = m(lin(X).float(), lin(Y).float(), SX, SY)
        torch.testing.assert_close(d, ref_d, atol=5e-2, rtol=5e-3)
        X.grad = None
    q = torch.randn(2, 3, 5, 8, device=DEV).requires_grad_()
    s = torch.randn(2, 6, 8, device=DEV)
    lin8 = torch.nn.Linear(8, 8).to(DEV)
    with torch.autocast("cuda", dtype=torch.float16):
        a = TF.jeanie(lin8(q), lin8(s), gamma=0.3, max_shift=1)
        b = TF.jeanie_from_cost(tw.euclidean_cost(lin8(q), lin8(s)), gamma=0.3, max_shift=1)
    assert a.dtype == torch.float32 and b.dtype == torch.float32
    (a.sum() + b.sum()).backward()
    assert torch.isfinite(q.grad).all()
