"""Edge sizes: an empty batch, long sequences, planes past 2 GiB, large batches.

The longest case is beyond what the float64 oracle finishes in seconds, so it
is checked by a size-independent property: the fused feature path (one
kernel family, 64 workgroups per pair) and the cost path on the materialised
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


def test_planes_past_2_gib_raise_value_error():
    """No length limit, but one pair's N x M planes are addressed with 32-bit
    byte offsets: 23200 x 23200 in float32 (2.15e9 bytes) is one past."""
    x, y = torch.rand(1, 23200, 1, device="cuda"), torch.rand(1, 23200, 1, device="cuda")
    s1 = torch.ones(1, 23200, 1, device="cuda")
    with pytest.raises(ValueError, match="below 2 GiB"):
        tw.UDTW()(x, y, s1, s1)


# ---- batches past 65535 pairs (the cost kernels index pairs in grid.y and
# launch in chunks; FVM folds the pair into grid.x). Pairs are independent, so
# the full batch must equal a float64 evaluation, and a slice of it must equal
# the same pairs computed alone, bit for bit.

BIG = 70000


def _maxnorm(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_pair_and_rbf_costs_past_65535_pairs(dtype):
    g = torch.Generator().manual_seed(21)
    A = torch.randn(BIG, 3, 5, generator=g, dtype=torch.float64)
    Bm = torch.randn(BIG, 4, 5, generator=g, dtype=torch.float64)
    tol = 1e-10 if dtype == torch.float64 else 1e-5
    for fn in (tw.squared_euclidean_cost, tw.rbf_cost):
        a = A.to("cuda", dtype).requires_grad_(True)
        b = Bm.to("cuda", dtype).requires_grad_(True)
        c = fn(a, b)
        w = torch.linspace(0.5, 1.5, c.numel(), device="cuda", dtype=dtype).view_as(c)
        (c * w).sum().backward()
        ar, br = A.clone().requires_grad_(True), Bm.clone().requires_grad_(True)
        if fn is tw.squared_euclidean_cost:
            cr = ((ar[:, :, None, :] - br[:, None, :, :]) ** 2).sum(-1)
        else:
            cr = (2 - 2 * torch.exp(-0.5 * (ar[:, :, None, :] - br[:, None, :, :]) ** 2)).sum(-1)
        (cr * w.double().cpu()).sum().backward()
        for got, want in ((c, cr), (a.grad, ar.grad), (b.grad, br.grad)):
            assert _maxnorm(got, want) < tol, fn.__name__
        # the last pairs alone: bitwise the batch's
        tail = fn(A[-7:].to("cuda", dtype), Bm[-7:].to("cuda", dtype))
        assert torch.equal(tail, c[-7:].detach())


def test_udtw_features_past_65535_pairs_and_normalize_past_21845():
    g = torch.Generator().manual_seed(22)
    for B, norm in ((BIG, False), (22000, True)):
        X = torch.randn(B, 3, 2, generator=g, dtype=torch.float64).cuda()
        Y = torch.randn(B, 3, 2, generator=g, dtype=torch.float64).cuda()
        sx = (0.5 + torch.rand(B, 3, 1, generator=g, dtype=torch.float64)).cuda()
        sy = (0.5 + torch.rand(B, 3, 1, generator=g, dtype=torch.float64)).cuda()
        m = tw.UDTW(gamma=0.5, beta=1.0, normalize=norm)
        d, p = m(X, Y, sx, sy)
        # the same pairs through the materialised-matrix path
        cost, pen, _ = TF.pairwise_matrices(X, Y, sx, sy, beta=1.0)
        dc, pc = TF.udtw_from_cost(cost, pen, gamma=0.5)
        if norm:
            for A_, S_ in ((X, sx), (Y, sy)):
                c2, p2, _ = TF.pairwise_matrices(A_, A_, S_, S_, beta=1.0)
                d2, q2 = TF.udtw_from_cost(c2, p2, gamma=0.5)
                dc, pc = dc - 0.5 * d2, pc - 0.5 * q2
        torch.testing.assert_close(d, dc, rtol=1e-10, atol=1e-10)
        torch.testing.assert_close(p, pc, rtol=1e-10, atol=1e-10)
        head = m(X[:5], Y[:5], sx[:5], sy[:5])
        assert torch.equal(head[0], d[:5]) and torch.equal(head[1], p[:5])


def test_jeanie_features_and_fvm_past_65535_pairs():
    g = torch.Generator().manual_seed(23)
    q = torch.randn(BIG, 2, 3, 4, generator=g, dtype=torch.float64).cuda()
    s = torch.randn(BIG, 3, 4, generator=g, dtype=torch.float64).cuda()
    d = TF.jeanie(q, s, gamma=0.3, max_shift=1)
    dc = TF.jeanie_from_cost(tw.euclidean_cost(q, s), gamma=0.3, max_shift=1)
    torch.testing.assert_close(d, dc, rtol=1e-10, atol=1e-10)
    c = torch.rand(BIG, 3, 4, 5, generator=g, dtype=torch.float64).cuda().requires_grad_(True)
    f = TF.fvm_from_cost(c, gamma=0.2)
    f.sum().backward()
    c5 = c[-5:].detach().clone().requires_grad_(True)
    f5 = TF.fvm_from_cost(c5, gamma=0.2)
    f5.sum().backward()
    assert torch.equal(f5, f[-5:].detach()) and torch.equal(c5.grad, c.grad[-5:])
    from oracle import jeanie as OJ
    cc = c[-3:].detach().cpu()
    torch.testing.assert_close(f[-3:].detach().cpu(), OJ.fvm_from_cost(cc, gamma=0.2),
                               rtol=1e-10, atol=1e-10)
