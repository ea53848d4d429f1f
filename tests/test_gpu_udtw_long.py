"""uDTW on sequences longer than one workgroup holds: several workgroups per
pair in both directions, and no length limit beyond one pair's 2 GiB planes.

Past 1024 rows (float32; 512 in float64) each pair runs ceil(N / 256)
workgroups of 256 rows. The forward hands each group's last row to the next
group through the R / P planes; the backward hands each group's first row
(E, Rbar, Pbar, A and the column gradient sums) to the group above through a
caller workspace. The arithmetic per cell and the order of every sum are
those of one workgroup per pair, so at lengths one workgroup still takes
(N <= 1024 in float32, 512 in float64) the results are compared bit for bit
with it (the launch layout is switched from the host with ``tw_test_set_mw``).
Beyond, the float64 oracle would take minutes, so size-independent properties
are checked instead.
"""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF
from torchwarp_amd import _hip

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


@pytest.fixture
def mw_mode():
    lib = _hip.library()
    yield lib.tw_test_set_mw
    lib.tw_test_set_mw(-1)


def _inputs(B, N, M, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)

    def walk(L):   # z-normalised random walks: modest costs along the best paths
        w = torch.cumsum(0.1 * torch.randn(B, L, D, generator=g, dtype=torch.float64), 1)
        return (w - w.mean(1, keepdim=True)) / w.std(1, keepdim=True)
    X, Y = walk(N), walk(M)
    sx = 0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64)
    sy = 0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64)
    return [t.to("cuda", dtype) for t in (X, Y, sx, sy)]


def _run(xs, gamma, beta, band):
    xs = [t.detach().clone().requires_grad_(True) for t in xs]
    d, p = tw.UDTW(gamma=gamma, beta=beta, bandwidth=band)(*xs)
    (d + 0.5 * p).sum().backward()
    torch.cuda.synchronize()
    return [d.detach(), p.detach()] + [t.grad for t in xs]


BITWISE = [  # (B, N, M, D, gamma, beta, band, dtype)
    (2, 1000, 1080, 1, 1.0, 1.0, None, torch.float32),   # D = 1, columns by DPP
    (2, 900, 1000, 3, 1.0, 1.0, None, torch.float32),    # D > 1: squared-distance plane
    (1, 500, 560, 1, 0.5, 1.0, None, torch.float64),     # float64
    (2, 1000, 990, 1, 1.0, 0.0, 80.0, torch.float32),    # soft-DTW with a band
    (1, 1000, 1010, 2, 0.1, 1.0, None, torch.float32),   # R in double precision
]


@pytest.mark.parametrize("case", BITWISE, ids=lambda c: "B{}N{}M{}D{}".format(*c[:4]))
def test_several_workgroups_equal_one_workgroup_bitwise(case, mw_mode):
    """Up to 1024 rows (512 in float64) one workgroup holds a pair at one row
    per thread, with the very arithmetic of the several-workgroup kernels:
    compared bit for bit (mode 1 splits every pair past 256 rows)."""
    B, N, M, D, gamma, beta, band, dtype = case
    xs = _inputs(B, N, M, D, dtype, seed=N + M)
    mw_mode(0)   # one workgroup per pair
    one = _run(xs, gamma, beta, band)
    mw_mode(1)   # several workgroups per pair in both directions
    many = _run(xs, gamma, beta, band)
    for k, (a, b) in enumerate(zip(one, many)):
        assert torch.equal(a, b), (case, k, (a - b).abs().max().item())
    assert all(torch.isfinite(t).all() for t in many)


def test_cost_path_several_workgroups_equal_one_workgroup_bitwise(mw_mode):
    g = torch.Generator().manual_seed(40)
    C = (3.0 * torch.rand(2, 1000, 1100, generator=g)).cuda()
    Q = (0.5 * torch.rand(2, 1000, 1100, generator=g)).cuda()

    def run():
        c, q = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
        d, p = TF.udtw_from_cost(c, q, gamma=2.0)
        (d + p).sum().backward()
        return [d.detach(), p.detach(), c.grad, q.grad]
    mw_mode(0)
    one = run()
    mw_mode(1)
    many = run()
    for a, b in zip(one, many):
        assert torch.equal(a, b)


def test_no_length_cap_at_20000_steps():
    """N = 20000, M = 20010 (past the reference's 16384-step limit), float32,
    one pair: 79 workgroups per pair in each direction. The problem is
    symmetric, and the feature kernels and the precomputed-cost kernels (two
    families) must agree."""
    N, M, gamma = 20000, 20010, 1.0
    x, y, sx, sy = _inputs(1, N, M, 1, torch.float32, seed=7)
    d1, p1, dx1, dy1, dsx1, dsy1 = _run([x, y, sx, sy], gamma, 1.0, None)
    # swapping the sequences gives the same bits
    d2, p2, dy2, dx2, dsy2, dsx2 = _run([y, x, sy, sx], gamma, 1.0, None)
    for a, b in ((d1, d2), (p1, p2), (dx1, dx2), (dy1, dy2), (dsx1, dsx2), (dsy1, dsy2)):
        assert torch.equal(a, b)
    assert all(torch.isfinite(t).all() for t in (d1, p1, dx1, dy1, dsx1, dsy1))
    cost, pen, _ = TF.pairwise_matrices(x, y, sx, sy, beta=1.0)
    d3, p3 = TF.udtw_from_cost(cost, pen, gamma=gamma)
    torch.testing.assert_close(d3, d1, rtol=1e-4, atol=0)
    torch.testing.assert_close(p3, p1, rtol=1e-4, atol=0)
    tw.check_async_status()


def test_path_field_identities_at_16000_steps_float64():
    """float64, N = 16000 (63 workgroups per pair): the gradient of the
    distance with respect to the cost is the path-probability field, in
    [0, 1] and exactly 1 at both corners (every path passes through them),
    and the penalty's gradient with respect to its matrix is the same field
    computed by the other adjoint recursion."""
    N, M = 16000, 16010
    g = torch.Generator().manual_seed(11)
    C = (3.0 * torch.rand(1, N, M, generator=g, dtype=torch.float64)).cuda()
    Q = (0.5 * torch.rand(1, N, M, generator=g, dtype=torch.float64)).cuda()
    c, q = C.requires_grad_(True), Q.requires_grad_(True)
    d, p = TF.udtw_from_cost(c, q, gamma=1.0)
    (E,) = torch.autograd.grad(d.sum(), c, retain_graph=True)
    (E2,) = torch.autograd.grad(p.sum(), q)
    assert float(E.min()) >= -1e-12 and float(E.max()) <= 1 + 1e-9
    assert abs(float(E[0, 0, 0]) - 1) < 1e-9 and abs(float(E[0, -1, -1]) - 1) < 1e-12
    torch.testing.assert_close(E2, E, rtol=0, atol=1e-12)
    tw.check_async_status()


def test_backward_wait_that_gives_up_is_reported():
    """The backward's hand-off wait, made to run out from the host: the
    gradients are NaN, the status is reported once, every kernel exits."""
    lib = _hip.library()
    tw.check_async_status()
    xs = [t.requires_grad_(True) for t in _inputs(1, 1100, 1150, 1, torch.float32, seed=3)]
    d, p = tw.UDTW(gamma=1.0, beta=1.0)(*xs)
    torch.cuda.synchronize()
    tw.check_async_status()   # the forward was fine
    lib.tw_test_set_wait(4, 1)
    try:
        (d + p).sum().backward()
        torch.cuda.synchronize()
    finally:
        lib.tw_test_set_wait(0, 0)
    assert torch.isnan(xs[0].grad).any()
    with pytest.raises(RuntimeError, match="gave up waiting"):
        tw.check_async_status()
    tw.check_async_status()


def test_fvm_past_one_workgroup_matches_oracle():
    """FVM's soft-DTW over sequences longer than one workgroup holds (float64,
    T = 600 > 512 rows): several workgroups per pair, against the oracle."""
    from oracle import jeanie as OJ
    g = torch.Generator().manual_seed(12)
    c = torch.rand(2, 3, 600, 640, generator=g, dtype=torch.float64)
    x = c.cuda().requires_grad_(True)
    d = TF.fvm_from_cost(x, gamma=0.3)
    d.sum().backward()
    want_d = OJ.fvm_from_cost(c, gamma=0.3)
    want_g = OJ.fvm_backward(c, torch.ones(2, dtype=torch.float64), 0.3)
    torch.testing.assert_close(d.detach().cpu(), want_d, rtol=1e-10, atol=1e-10)
    err = ((x.grad.cpu() - want_g).abs().max() / want_g.abs().max()).item()
    assert err < 1e-10, err
    tw.check_async_status()
