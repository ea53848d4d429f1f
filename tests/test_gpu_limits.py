"""Edge sizes: an empty batch, the longest sequences this build takes, one past.

The longest case is beyond what the float64 oracle finishes in seconds, so it
is checked by a size-independent property: the fused feature path (one
kernel family, 16 rows per thread) and the cost path on the materialised
matrices (another kernel family) must agree, and swapping the sequences
must not change the result.
"""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def test_empty_batch():
    X, Y = torch.rand(0, 7, 2, device="cuda"), torch.rand(0, 9, 2, device="cuda")
    S1, S2 = torch.ones(0, 7, 1, device="cuda"), torch.ones(0, 9, 1, device="cuda")
    xs = [t.requires_grad_(True) for t in (X, Y, S1, S2)]
    d, p = tw.UDTW(gamma=0.5)(*xs)
    assert d.shape == (0,) and p.shape == (0,)
    (d.sum() + p.sum()).backward()
    assert xs[0].grad.shape == X.shape
    c = torch.rand(0, 2, 5, 6, device="cuda", requires_grad=True)
    out = TF.jeanie_from_cost(c, gamma=0.1)
    assert out.shape == (0,)
    out.sum().backward()
    assert c.grad.shape == c.shape
    q, s = torch.rand(0, 3, 4, 8, device="cuda"), torch.rand(0, 5, 8, device="cuda")
    assert TF.jeanie(q, s, gamma=0.1).shape == (0,)
    assert TF.fvm_from_cost(torch.rand(0, 3, 4, 5, device="cuda"), gamma=0.1).shape == (0,)
    cost = torch.rand(0, 4, 6, device="cuda", requires_grad=True)
    d, p = TF.udtw_from_cost(cost, torch.zeros_like(cost), gamma=0.3)
    (d.sum() + p.sum()).backward()
    assert tw.rbf_cost(q, s).shape == (0, 3, 4, 5)


def test_longest_sequences_agree_across_kernel_families():
    g = torch.Generator().manual_seed(15)
    N, M = 16384, 16400
    x = torch.cumsum(0.05 * torch.randn(1, N, 1, generator=g), 1).cuda()
    y = torch.cumsum(0.05 * torch.randn(1, M, 1, generator=g), 1).cuda()
    sx = (0.5 + torch.rand(1, N, 1, generator=g)).cuda()
    sy = (0.5 + torch.rand(1, M, 1, generator=g)).cuda()
    d1, p1 = tw.UDTW(gamma=1.0, beta=1.0)(x, y, sx, sy)
    d2, p2 = tw.UDTW(gamma=1.0, beta=1.0)(y, x, sy, sx)   # swapped
    cost, pen, _ = TF.pairwise_matrices(x, y, sx, sy, beta=1.0)
    d3, p3 = TF.udtw_from_cost(cost, pen, gamma=1.0)
    torch.testing.assert_close(d1, d2, rtol=0, atol=0)
    torch.testing.assert_close(p1, p2, rtol=0, atol=0)
    torch.testing.assert_close(d1, d3, rtol=1e-4, atol=1e-3)
    torch.testing.assert_close(p1, p3, rtol=1e-4, atol=1e-3)


def test_one_past_the_longest_raises():
    x, y = torch.rand(1, 16385, 1, device="cuda"), torch.rand(1, 16390, 1, device="cuda")
    s1, s2 = torch.ones(1, 16385, 1, device="cuda"), torch.ones(1, 16390, 1, device="cuda")
    with pytest.raises((RuntimeError, ValueError), match="16384"):
        tw.UDTW()(x, y, s1, s2)
