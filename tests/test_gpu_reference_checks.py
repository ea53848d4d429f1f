"""Remaining checks of the reference's tests/test_udtw.py:117-250 and
tests/test_jeanie.py:311-353, on the HIP path: finite-difference gradchecks
(band, fused features), one output used, and input validation with the
reference's exception types."""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF
from torchwarp_amd.jeanie.functional import _jeanie_dp_features

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"
F64 = dict(dtype=torch.float64, device=DEV)


def _inputs(B, N, M, D=3):
    g = torch.Generator().manual_seed(16)
    return [t.to(DEV) for t in (torch.rand(B, N, D, generator=g, dtype=torch.float64),
                                torch.rand(B, M, D, generator=g, dtype=torch.float64),
                                0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64),
                                0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64))]


def test_gradcheck_with_band():
    cost = torch.rand(2, 6, 6, **F64).requires_grad_()
    pen = torch.randn(2, 6, 6, **F64).requires_grad_()
    fn = lambda c, p: TF.udtw_from_cost(c, p, gamma=0.3, bandwidth=1)
    assert torch.autograd.gradcheck(fn, (cost, pen))


def test_fused_gradcheck():
    X, Y, SX, SY = [t.requires_grad_() for t in _inputs(2, 4, 6)]
    assert torch.autograd.gradcheck(tw.UDTW(gamma=0.3, beta=0.8), (X, Y, SX, SY))


@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean"])
def test_fused_features_gradcheck(metric):
    q = torch.randn(2, 2, 2, 4, 3, **F64).requires_grad_()
    s = torch.randn(2, 5, 3, **F64).requires_grad_()
    fn = lambda q, s: _jeanie_dp_features(q, s, 0.5, 1, 1, metric, "auto")[0]
    assert torch.autograd.gradcheck(fn, (q, s))


def test_only_one_output_used():
    X, Y, SX, SY = [t.requires_grad_(True) for t in _inputs(2, 4, 5)]
    dist, _ = tw.UDTW(gamma=0.1)(X, Y, SX, SY)
    dist.sum().backward()
    assert torch.isfinite(X.grad).all() and torch.isfinite(SX.grad).all()


def test_input_validation():
    X, Y, SX, SY = _inputs(2, 4, 5)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.0)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1, beta=-1.0)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1)(X[0], Y, SX, SY)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1)(X[0], Y[0], SX[0], SY[0])
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1, backend="nope")
    r = lambda *s: torch.rand(*s, device=DEV)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(r(4, 5), gamma=0.1)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(r(2, 4, 5), gamma=0.1)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(r(1, 2, 4, 5), gamma=0.0)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(r(1, 2, 4, 5), gamma=0.1, max_shift=-1)
    with pytest.raises(ValueError):
        TF.jeanie(r(2, 4, 3), r(5, 3))
    with pytest.raises(TypeError):
        TF.soft_dtw_from_cost(torch.ones(1, 3, 3, dtype=torch.int64, device=DEV))
    with pytest.raises(ValueError):
        TF.soft_dtw_from_cost(r(3, 3))
    with pytest.raises(ValueError):
        TF.fvm_from_cost(r(4, 5, 6))
    with pytest.raises(TypeError):
        TF.jeanie_from_cost(r(1, 2, 4, 5), 0.1)
