"""normalize=True with N == M runs the three divergence terms as one 3B-pair launch.

Each pair is computed independently, so the batched values must equal those of
three separate calls (bitwise for the distances; gradients to float64
rounding, since autograd adds X's two contributions in another order).
"""

import pytest
import torch

import torchwarp_amd as tw

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def _leaves(*shapes, seed=3):
    g = torch.Generator().manual_seed(seed)
    out = []
    for shape, pos in shapes:
        t = 0.5 + torch.rand(*shape, generator=g, dtype=torch.float64) if pos else \
            torch.randn(*shape, generator=g, dtype=torch.float64)
        out.append(t.cuda().requires_grad_(True))
    return out


@pytest.mark.parametrize("D", [1, 6])
def test_udtw_normalize_batched_equals_separate(D):
    X, Y, sx, sy = _leaves(((4, 17, D), 0), ((4, 17, D), 0), ((4, 17, 1), 1), ((4, 17, 1), 1))
    m = tw.UDTW(gamma=0.4, beta=0.8)
    d, p = tw.UDTW(gamma=0.4, beta=0.8, normalize=True)(X, Y, sx, sy)
    gb = torch.autograd.grad((d + 2 * p).sum(), (X, Y, sx, sy))
    dxy, pxy = m(X, Y, sx, sy)
    dxx, pxx = m(X, X, sx, sx)
    dyy, pyy = m(Y, Y, sy, sy)
    d2, p2 = dxy - 0.5 * (dxx + dyy), pxy - 0.5 * (pxx + pyy)
    gs = torch.autograd.grad((d2 + 2 * p2).sum(), (X, Y, sx, sy))
    assert torch.equal(d, d2) and torch.equal(p, p2)
    for a, b in zip(gb, gs):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_soft_dtw_normalize_batched_equals_separate():
    X, Y = _leaves(((3, 21, 4), 0), ((3, 21, 4), 0))
    d = tw.SoftDTW(gamma=0.3, normalize=True)(X, Y)
    gb = torch.autograd.grad(d.sum(), (X, Y))
    m = tw.SoftDTW(gamma=0.3)
    d2 = m(X, Y) - 0.5 * (m(X, X) + m(Y, Y))
    gs = torch.autograd.grad(d2.sum(), (X, Y))
    assert torch.equal(d, d2)
    for a, b in zip(gb, gs):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
