"""Optimal (gamma = 0) paths on the GPU against the oracle's restatement of
the reference scan (paths.py:85-127), compared with ``==`` (bit-exact
indices), and the soft path matrices of ``torchwarp_amd.paths`` against the
float64 oracle gradients.

Integer-valued costs make exact ties common, which exercises the strict
``<`` scan order (viewpoints ascending, then (t-1,u-1), (t-1,u), (t,u-1)) and
the first-minimum end viewpoint.
"""

import pytest
import torch

from oracle import jeanie as OJ, paths as OP
import torchwarp_amd as tw

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"


def _costs(seed, shape, ties):
    g = torch.Generator().manual_seed(seed)
    if ties:
        return torch.randint(0, 3, shape, generator=g).double()
    return torch.rand(shape, generator=g, dtype=torch.float64)


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("shape", [(3, 6, 7), (2, 1, 5), (2, 5, 1), (1, 1, 1), (2, 9, 4)])
def test_optimal_path_2d(shape, ties):
    c = _costs(sum(shape) + ties, shape, ties)
    assert tw.paths.optimal_path(c.to(DEV)) == OP.optimal_path(c.numpy())


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("shape,shift,start", [
    ((2, 4, 5, 6), 1, None), ((2, 5, 6, 4), 2, None), ((1, 3, 4, 4), 0, None),
    ((2, 4, 5, 5), 1, 2), ((2, 4, 5, 5), 0, 1), ((1, 6, 3, 7), 6, None), ((1, 4, 5, 5), 1, -1),
])
def test_optimal_path_viewpoints(shape, shift, start, ties):
    c = _costs(sum(shape) + shift + ties, shape, ties)
    got = tw.paths.optimal_path(c.to(DEV), max_shift=shift, start_view=start)
    sv = None if start is None else start % shape[1]
    assert got == OP.optimal_path(c.numpy(), max_shift=shift, start_view=sv)


def test_float32_cost_is_evaluated_in_float64():
    c = _costs(7, (2, 5, 6), False).float()
    assert tw.paths.optimal_path(c.to(DEV)) == OP.optimal_path(c.double().numpy())


def test_soft_dtw_alignment_matches_oracle():
    c = _costs(3, (2, 6, 7), False)
    a = tw.paths.soft_dtw(c.to(DEV), gamma=0.1)
    ref = c.clone().requires_grad_(True)
    d = OJ.soft_dtw_from_cost(ref, gamma=0.1)
    (g,) = torch.autograd.grad(d.sum(), ref)
    assert torch.allclose(a.distance.cpu(), d.detach(), rtol=1e-10, atol=1e-12)
    assert torch.allclose(a.path_matrix.cpu(), g, rtol=1e-10, atol=1e-12)
    assert a.optimal_path == OP.optimal_path(c.numpy())


def test_jeanie_alignment_paths():
    g = torch.Generator().manual_seed(11)
    q = torch.randn(2, 4, 5, 3, generator=g, dtype=torch.float64)
    s = torch.randn(2, 6, 3, generator=g, dtype=torch.float64)
    a = tw.paths.jeanie(q.to(DEV), s.to(DEV), gamma=0.1, max_shift=1, start_view=2)
    D = OJ.euclidean_cost(q, s)
    assert a.optimal_path == OP.optimal_path(D.numpy(), max_shift=1, start_view=2)
    assert all(p[0][2] == 2 for p in a.optimal_path)
    assert a.path_matrix.shape == (2, 4, 5, 6)
    with pytest.raises(NotImplementedError):
        a.plot()
