"""HIP kernels through the public API vs the official implementation's golden outputs.

Mirrors the reference's own golden tests (``tests/test_udtw.py``,
``tests/test_jeanie.py``): the same cases, float64 on the GPU, compared at
atol 1e-10 / rtol 1e-9.
"""

import pytest
import torch

import golden_cases as G
from golden_cases import golden
import torchwarp_amd as tw
import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"


def close(a, b, tol=1e-10):
    torch.testing.assert_close(a.detach().cpu(), b, atol=tol, rtol=1e-9)


def _udtw_run(module, inputs):
    xs = [x.detach().to(DEV).requires_grad_(True) for x in inputs]
    d, p = module(*xs)
    (d.sum() + 2.0 * p.sum()).backward()
    return [d, p] + [x.grad for x in xs]


@pytest.mark.parametrize("N,M", G.UDTW_SHAPES)
@pytest.mark.parametrize("gamma", G.GAMMAS)
@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("method", ["gemm", "diff"])
def test_udtw_matches(N, M, gamma, normalize, method):
    ref = golden("udtw.matches", N=N, M=M, gamma=gamma, normalize=normalize)
    got = _udtw_run(tw.UDTW(gamma=gamma, beta=0.7, normalize=normalize, method=method),
                    ref["inputs"])
    for a, b in zip(got, ref["outputs"]):
        close(a, b)


@pytest.mark.parametrize("N,M,bandwidth", G.UDTW_BANDS)
def test_udtw_bandwidth(N, M, bandwidth):
    ref = golden("udtw.bandwidth", N=N, M=M, bandwidth=bandwidth)
    got = _udtw_run(tw.UDTW(gamma=0.1, beta=0.7, bandwidth=bandwidth), ref["inputs"])
    for a, b in zip(got, ref["outputs"]):
        close(a, b)


@pytest.mark.parametrize("beta", G.UDTW_BETAS)
def test_udtw_beta(beta):
    ref = golden("udtw.beta", beta=beta)
    got = _udtw_run(tw.UDTW(gamma=0.1, beta=beta), ref["inputs"])
    for a, b in zip(got, ref["outputs"]):
        close(a, b)


def test_udtw_large():
    ref = golden("udtw.large", B=2, N=40, M=50)
    got = _udtw_run(tw.UDTW(gamma=0.1, beta=0.7), ref["inputs"])
    for a, b in zip(got, ref["outputs"]):
        close(a, b)


def test_udtw_float32_accuracy():
    """float32 against the float64 truth as max-normalised error (D = 32: the
    pairwise-cost kernel + squared-distance DP path)."""
    ref = golden("udtw.float32")
    got = _udtw_run(tw.UDTW(gamma=0.1, beta=0.7), [x.float() for x in ref["inputs"]])
    for k, (a, b) in enumerate(zip(got, ref["outputs"])):
        err = ((a.detach().double().cpu() - b).abs().max() / b.abs().max()).item()
        assert err < (1e-5 if k < 2 else 1e-3), (k, err)


def test_udtw_unreachable_band_raises():
    X, Y = torch.rand(1, 3, 5, device=DEV), torch.rand(1, 9, 5, device=DEV)
    S1, S2 = torch.ones(1, 3, 1, device=DEV), torch.ones(1, 9, 1, device=DEV)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1, bandwidth=2)(X, Y, S1, S2)


def test_pairwise_matrices_golden():
    ref = golden("udtw.pairwise_matrices")
    for method in ("gemm", "diff"):
        got = TF.pairwise_matrices(*[x.to(DEV) for x in ref["inputs"]], beta=0.5, method=method)
        for a, b in zip(got, ref["outputs"]):
            torch.testing.assert_close(a.cpu(), b, atol=1e-12, rtol=1e-10)


def _value_and_grad(fn, cost):
    c = cost.detach().to(DEV).requires_grad_(True)
    out = fn(c)
    out.sum().backward()
    return out, c.grad


@pytest.mark.parametrize("T,U", G.SDTW_SHAPES)
@pytest.mark.parametrize("gamma", G.GAMMAS)
def test_soft_dtw(T, U, gamma):
    ref = golden("jeanie.soft_dtw", T=T, U=U, gamma=gamma)
    v, g = _value_and_grad(lambda c: TF.soft_dtw_from_cost(c[None], gamma=gamma)[0], ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])


@pytest.mark.parametrize("K,T,U", G.JEANIE_1D_SHAPES)
@pytest.mark.parametrize("shift", G.JEANIE_1D_SHIFTS)
def test_jeanie_1d(K, T, U, shift):
    ref = golden("jeanie.jeanie_1d", K=K, T=T, U=U, shift=shift)
    v, g = _value_and_grad(
        lambda c: TF.jeanie_from_cost(c[None], gamma=0.1, max_shift=shift)[0], ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])
    _, acc = TF.jeanie_from_cost(ref["cost"][None].to(DEV), gamma=0.1, max_shift=shift,
                                 return_accumulator=True)
    close(acc[0], ref["accumulator"])


@pytest.mark.parametrize("K1,K2,T,U", G.JEANIE_2D_SHAPES)
@pytest.mark.parametrize("s_az,s_alt", G.JEANIE_2D_SHIFTS)
def test_jeanie_2d(K1, K2, T, U, s_az, s_alt):
    ref = golden("jeanie.jeanie_2d", K1=K1, K2=K2, T=T, U=U, s_az=s_az, s_alt=s_alt)
    v, g = _value_and_grad(
        lambda c: TF.jeanie_from_cost(c[None], gamma=0.1, max_shift=(s_az, s_alt))[0],
        ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])


def test_jeanie_batched():
    ref = golden("jeanie.batched")
    close(TF.jeanie_from_cost(ref["cost_1d"].to(DEV), gamma=0.1, max_shift=1), ref["value_1d"])
    close(TF.jeanie_from_cost(ref["cost_2d"].to(DEV), gamma=0.1, max_shift=(1, 1)),
          ref["value_2d"])


@pytest.mark.parametrize("name,shape", G.FVM_CASES)
def test_fvm(name, shape):
    ref = golden("jeanie.fvm", name=name)
    v, g = _value_and_grad(lambda c: TF.fvm_from_cost(c[None], gamma=0.1)[0], ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])
    close(TF.fvm_from_cost(ref["batch"].to(DEV), gamma=0.1), ref["batch_value"])


def _large_fn(name, shift):
    if name == "soft_dtw":
        return lambda c: TF.soft_dtw_from_cost(c[None], gamma=0.1)[0]
    if name.startswith("fvm"):
        return lambda c: TF.fvm_from_cost(c[None], gamma=0.1)[0]
    return lambda c: TF.jeanie_from_cost(c[None], gamma=0.1, max_shift=shift)[0]


@pytest.mark.parametrize("name,shape,shift", G.LARGE_COST)
def test_large(name, shape, shift):
    ref = golden("jeanie.large", name=name, shape=shape)
    v, g = _value_and_grad(_large_fn(name, shift), ref["cost"])
    close(v, ref["value"])
    close(g, ref["grad"])


@pytest.mark.parametrize("name", G.DISTANCES)
def test_distances(name):
    ref = golden("jeanie.distance", name=name)
    q = ref["q"].to(DEV).requires_grad_()
    s = ref["s"].to(DEV).requires_grad_()
    out = getattr(tw, name)(q, s)
    close(out, ref["value"])
    for a, b in zip(torch.autograd.grad(out.sum(), (q, s)), ref["grads"]):
        close(a, b)
    close(getattr(tw, name)(ref["qb"].to(DEV), ref["sb"].to(DEV)), ref["batch_value"])


def test_end_to_end():
    ref = golden("jeanie.end_to_end")
    q, s = ref["q"].to(DEV).requires_grad_(), ref["s"].to(DEV).requires_grad_()
    d = TF.jeanie_from_cost(tw.euclidean_cost(q[None], s[None]), gamma=0.1, max_shift=1)[0]
    close(d, ref["value"])
    for a, b in zip(torch.autograd.grad(d, (q, s)), ref["grads"]):
        close(a, b)


@pytest.mark.parametrize("metric", G.METRICS)
@pytest.mark.parametrize("K,T,U,shift", G.FEATURES_1D)
def test_jeanie_features_1d(metric, K, T, U, shift):
    ref = golden("jeanie.features_1d", metric=metric, K=K, T=T, U=U, shift=shift)
    q, s = ref["q"].to(DEV).requires_grad_(), ref["s"].to(DEV).requires_grad_()
    d = TF.jeanie(q, s, gamma=0.1, max_shift=shift, metric=metric)
    close(d, ref["value"])
    for a, b in zip(torch.autograd.grad(d.sum(), (q, s)), ref["grads"]):
        close(a, b)


@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean"])
def test_jeanie_features_2d(metric):
    ref = golden("jeanie.features_2d", metric=metric)
    q, s = ref["q"].to(DEV).requires_grad_(), ref["s"].to(DEV).requires_grad_()
    d, acc = TF.jeanie(q, s, gamma=0.1, max_shift=(1, 1), metric=metric, return_accumulator=True)
    close(d, ref["value"])
    for a, b in zip(torch.autograd.grad(d.sum(), (q, s)), ref["grads"]):
        close(a, b)
    close(acc[0], ref["accumulator"])


@pytest.mark.parametrize("K,T,U,shift", G.ACCUMULATOR_COST)
def test_accumulator_cost(K, T, U, shift):
    ref = golden("parity.accumulator_cost", K=K, T=T, U=U, shift=shift)
    c = ref["cost"].to(DEV).requires_grad_()
    d, R = TF.jeanie_from_cost(c[None], gamma=0.3, max_shift=shift, return_accumulator=True)
    g = torch.autograd.grad(d[0] + 0.1 * (R ** 2).mean(), c)[0]
    close(g, ref["grad"], tol=1e-9)


def test_accumulator_2d():
    ref = golden("parity.accumulator_2d")
    c = ref["cost"].to(DEV).requires_grad_()
    d, R = TF.jeanie_from_cost(c[None], gamma=0.3, max_shift=(1, 1), return_accumulator=True)
    g = torch.autograd.grad(d[0] + R.sin().sum(), c)[0]
    close(g, ref["grad"], tol=1e-9)


@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean"])
def test_accumulator_features(metric):
    ref = golden("parity.accumulator_features", metric=metric)
    q, s = ref["q"].to(DEV).requires_grad_(), ref["s"].to(DEV).requires_grad_()
    d, R = TF.jeanie(q[None], s[None], gamma=0.3, max_shift=1, metric=metric,
                     return_accumulator=True)
    for a, b in zip(torch.autograd.grad(d[0] + 0.1 * (R ** 2).mean(), (q, s)), ref["grads"]):
        close(a, b, tol=1e-9)


def test_features_zero_distance_grad_is_finite():
    q = torch.ones(1, 2, 3, 4, dtype=torch.float64, device=DEV, requires_grad=True)
    s = torch.ones(1, 3, 4, dtype=torch.float64, device=DEV, requires_grad=True)
    TF.jeanie(q, s, gamma=0.1, max_shift=1).sum().backward()
    assert torch.isfinite(q.grad).all() and torch.isfinite(s.grad).all()
