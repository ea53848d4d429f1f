"""uDTW launch layouts for longer and ragged sequences against the float64 oracle.

The launcher gives one row per thread up to 1024 rows (512 in float64), with
the column operands in LDS up to 256 rows and travelling by DPP beyond, then
several rows per thread. For D > 1 the squared distances and their adjoint
sit diagonal-major between the pair-cost kernels and the sweeps. These
shapes put each layout (N just past 256, 512 and 1024; N > M, which the API
swaps; D = 1 and D > 1; the precomputed-cost path) under the forward and
the backward.
"""

import pytest
import torch

from oracle import udtw as OU
import torchwarp_amd as tw
import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

SHAPES = [  # (B, N, M, D, gamma)
    (2, 300, 310, 1, 1.0),
    (2, 290, 270, 4, 1.0),     # N > M: the API swaps the sequences
    (1, 600, 640, 8, 1.0),     # one row per thread in float32, two in float64
    (2, 250, 260, 4, 1.0),     # ragged row and column tails of the cost tiles
    (1, 64, 1000, 4, 1.0),     # few rows against long columns
    (2, 150, 170, 3, 1.0),     # D not a multiple of 4: single-element cost loads
    (1, 100, 130, 75, 1.0),    # D > 64: cost kernels in feature slices (64 float32, 32 float64)
    (1, 1100, 1030, 1, 1.0),   # beyond 1024 rows: several rows per thread
]


def _maxnorm(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}N{}M{}D{}".format(*s[:4]))
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_udtw_features_layouts(shape, dtype):
    B, N, M, D, gamma = shape
    g = torch.Generator().manual_seed(5)
    X = torch.randn(B, N, D, generator=g, dtype=torch.float64) / D ** 0.5
    Y = torch.randn(B, M, D, generator=g, dtype=torch.float64) / D ** 0.5
    sx = 0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64)
    sy = 0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64)
    xs = [t.to("cuda", dtype).requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = tw.UDTW(gamma=gamma, beta=1.0)(*xs)
    (d + p).sum().backward()
    ref = [t.clone().requires_grad_(True) for t in (X, Y, sx, sy)]
    rd, rp = OU.udtw(*ref, gamma=gamma, beta=1.0)
    (rd + rp).sum().backward()
    got = [d, p] + [t.grad for t in xs]
    want = [rd, rp] + [t.grad for t in ref]
    errs = [_maxnorm(a, b) for a, b in zip(got, want)]
    if dtype == torch.float64:
        assert max(errs) < 1e-9, errs
    else:
        assert max(errs[:2]) < 1e-5, errs
        assert max(errs[2:]) < 2e-3, errs


@pytest.mark.parametrize("NM", [(300, 330), (700, 650)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_udtw_cost_layouts(NM, dtype):
    N, M = NM
    g = torch.Generator().manual_seed(6)
    C = torch.rand(2, N, M, generator=g, dtype=torch.float64)
    Q = 0.2 * torch.rand(2, N, M, generator=g, dtype=torch.float64)
    c, q = C.to("cuda", dtype).requires_grad_(True), Q.to("cuda", dtype).requires_grad_(True)
    d, p = TF.udtw_from_cost(c, q, gamma=0.5)
    (d + 3 * p).sum().backward()
    rc, rq = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    rd, rp = OU.udtw_from_cost(rc, rq, gamma=0.5)
    (rd + 3 * rp).sum().backward()
    errs = [_maxnorm(a, b) for a, b in zip([d, p, c.grad, q.grad], [rd, rp, rc.grad, rq.grad])]
    if dtype == torch.float64:
        assert max(errs) < 1e-9, errs
    else:
        assert max(errs[:2]) < 1e-5, errs
        # d cost carries the penalty coupling -Pbar (P_k - A_s) / gamma: P
        # accumulates ~N + M penalties with float32 softmax weights, so each P
        # is off by ~1e-7 |P|, and differences of P divided by gamma reach the
        # cost gradient (measured 2.1e-3 at 700 x 650, gamma 0.5, penalty
        # weight 3; 2.3e-5 without the penalty). R is kept in double here.
        assert max(errs[2:]) < 3e-3, errs


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_feat_bwd_with_and_without_forward_plane(dtype):
    """tw_udtw_feat_bwd reads the forward's squared distances when given its
    workspace and recomputes them when given NULL: both give the same bits."""
    from torchwarp_amd import _hip
    B, N, M, D = 3, 70, 90, 5
    g = torch.Generator().manual_seed(8)
    X, Y = (torch.randn(B, L, D, generator=g, dtype=dtype).cuda() for L in (N, M))
    vx, vy = (0.5 + torch.rand(B, L, generator=g, dtype=dtype).cuda() for L in (N, M))
    R = X.new_empty(B, _hip.carry_cols(N, M, 0.7, dtype))
    P = X.new_empty(B, N * M)
    o1, o2 = X.new_empty(B), X.new_empty(B)
    nws = _hip.udtw_workspace_elems(B, N, M, D, dtype)
    wsb = nws * X.element_size()
    S = X.new_empty(nws)
    _hip.call("tw_udtw_feat_fwd", dtype, X, Y, vx, vy, B, N, M, D, 0.7, 1.0, 1e-8, 0.0, 1,
              R, P, o1, o2, S, wsb)
    gr = torch.rand(B, generator=g, dtype=dtype).cuda()
    outs = []
    for fwd_ws in (S, None):
        grads = [torch.empty_like(t) for t in (X, Y, vx, vy)]
        _hip.call("tw_udtw_feat_bwd", dtype, X, Y, vx, vy, R, P, gr, gr, B, N, M, D, 0.7, 1.0,
                  1e-8, 0.0, 1, 1, *grads, fwd_ws, X.new_empty(nws), wsb)
        outs.append(grads)
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


BANDS = [  # (B, N, M, D, bandwidth): blocks of whole wavefronts outside the band are skipped
    (2, 300, 310, 1, 25.0),     # rows travel by DPP (N > 256)
    (1, 600, 640, 8, 40.0),     # D > 1: diagonal-major S / dS
    (2, 200, 220, 3, 21.5),     # columns in LDS (N <= 256)
    (1, 1100, 1030, 1, 90.0),   # several rows per thread
]


@pytest.mark.parametrize("shape", BANDS, ids=lambda s: "B{}N{}M{}D{}w{}".format(*s))
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_udtw_band_layouts(shape, dtype):
    """Sakoe-Chiba band |i - j| <= bandwidth (udtw_cuda.cu:126-130) on long
    sequences, where most wavefront blocks lie outside the band."""
    B, N, M, D, band = shape
    g = torch.Generator().manual_seed(10)
    X = torch.randn(B, N, D, generator=g, dtype=torch.float64) / D ** 0.5
    Y = torch.randn(B, M, D, generator=g, dtype=torch.float64) / D ** 0.5
    sx = 0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64)
    sy = 0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64)
    xs = [t.to("cuda", dtype).requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = tw.UDTW(gamma=0.5, beta=1.0, bandwidth=band)(*xs)
    (d + p).sum().backward()
    ref = [t.clone().requires_grad_(True) for t in (X, Y, sx, sy)]
    rd, rp = OU.udtw(*ref, gamma=0.5, beta=1.0, bandwidth=band)
    (rd + rp).sum().backward()
    errs = [_maxnorm(a, b) for a, b in zip([d, p] + [t.grad for t in xs],
                                           [rd, rp] + [t.grad for t in ref])]
    if dtype == torch.float64:
        assert max(errs) < 1e-9, errs
    else:
        assert max(errs[:2]) < 1e-5, errs
        assert max(errs[2:]) < 2e-3, errs


def test_udtw_cost_band_long():
    g = torch.Generator().manual_seed(11)
    C = torch.rand(2, 700, 650, generator=g, dtype=torch.float64)
    Q = 0.2 * torch.rand(2, 700, 650, generator=g, dtype=torch.float64)
    c, q = C.cuda().requires_grad_(True), Q.cuda().requires_grad_(True)
    d, p = TF.udtw_from_cost(c, q, gamma=0.5, bandwidth=60)
    (d + 3 * p).sum().backward()
    rc, rq = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    rd, rp = OU.udtw_from_cost(rc, rq, gamma=0.5, bandwidth=60)
    (rd + 3 * rp).sum().backward()
    errs = [_maxnorm(a, b) for a, b in zip([d, p, c.grad, q.grad], [rd, rp, rc.grad, rq.grad])]
    assert max(errs) < 1e-9, errs


@pytest.mark.parametrize("B,N,M", [(3, 700, 720), (260, 300, 310)])
def test_udtw_many_groups_and_large_batch(B, N, M):
    """D = 1 forward with several workgroups per pair (B = 3: three groups
    each) and, past the workgroup budget (B = 260: 520 groups), one
    workgroup per pair; float64 against the oracle."""
    g = torch.Generator().manual_seed(14)
    X = torch.randn(B, N, 1, generator=g, dtype=torch.float64)
    Y = torch.randn(B, M, 1, generator=g, dtype=torch.float64)
    sx = 0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64)
    sy = 0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64)
    xs = [t.cuda().requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = tw.UDTW(gamma=1.0, beta=0.5)(*xs)
    (d + p).sum().backward()
    ref = [t.clone().requires_grad_(True) for t in (X, Y, sx, sy)]
    rd, rp = OU.udtw(*ref, gamma=1.0, beta=0.5)
    (rd + rp).sum().backward()
    errs = [_maxnorm(a, b) for a, b in zip([d, p] + [t.grad for t in xs],
                                           [rd, rp] + [t.grad for t in ref])]
    assert max(errs) < 1e-9, errs


# float32 with R carried in double precision: long sequences at a small gamma
# ((N + M - 1) log2(e) / gamma > 2048). Every one-row layout: LDS columns
# (N <= 256), columns by DPP with several workgroups per pair in the forward,
# the squared-distance plane (D > 1) and the precomputed-cost path. Without
# double R these shapes carry 1e-2 .. 5e-2 relative gradient error.
RD_SHAPES = [  # (B, N, M, D, gamma)
    (2, 200, 230, 1, 0.05),
    (1, 700, 720, 1, 0.05),
    (2, 300, 320, 4, 0.05),
]


@pytest.mark.parametrize("shape", RD_SHAPES, ids=lambda s: "B{}N{}M{}D{}".format(*s[:4]))
def test_float32_with_double_r_matches_float64(shape):
    from torchwarp_amd import _hip
    B, N, M, D, gamma = shape
    assert _hip.carry_cols(N, M, gamma, torch.float32) == 2 * N * M
    g = torch.Generator().manual_seed(9)
    X = torch.randn(B, N, D, generator=g, dtype=torch.float64)
    Y = torch.randn(B, M, D, generator=g, dtype=torch.float64)
    sx = 0.5 + torch.rand(B, N, 1, generator=g, dtype=torch.float64)
    sy = 0.5 + torch.rand(B, M, 1, generator=g, dtype=torch.float64)
    xs = [t.to("cuda", torch.float32).requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = tw.UDTW(gamma=gamma, beta=1.0)(*xs)
    (d + p).sum().backward()
    ref = [t.clone().requires_grad_(True) for t in (X, Y, sx, sy)]
    rd, rp = OU.udtw(*ref, gamma=gamma, beta=1.0)
    (rd + rp).sum().backward()
    errs = [_maxnorm(a, b) for a, b in zip([d, p] + [t.grad for t in xs],
                                            [rd, rp] + [t.grad for t in ref])]
    print("\nfloat32, double R, {}: errors {}".format(shape, ["%.2e" % e for e in errs]))
    assert max(errs[:2]) < 1e-5, errs
    # feature gradients measured 3e-5 .. 5e-4; the sigma gradients carry the
    # penalty coupling through float32 P (measured up to 1.1e-3)
    assert max(errs[2:4]) < 1e-3, errs
    assert max(errs[4:]) < 2e-3, errs


def test_float32_cost_path_with_double_r_matches_float64():
    g = torch.Generator().manual_seed(10)
    C = 3.0 * torch.rand(2, 500, 520, generator=g, dtype=torch.float64)
    Q = 0.5 * torch.rand(2, 500, 520, generator=g, dtype=torch.float64)
    c, q = (t.to("cuda", torch.float32).requires_grad_(True) for t in (C, Q))
    d, p = TF.udtw_from_cost(c, q, gamma=0.05)
    (d + p).sum().backward()
    cr, qr = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    rd, rp = OU.udtw_from_cost(cr, qr, gamma=0.05)
    (rd + rp).sum().backward()
    errs = [_maxnorm(a, b) for a, b in zip([d, p, c.grad, q.grad], [rd, rp, cr.grad, qr.grad])]
    print("\nfloat32 cost path, double R: errors", ["%.2e" % e for e in errs])
    assert max(errs[:2]) < 1e-5, errs
    # d penalty measured 2e-6; d cost carries the penalty coupling through
    # float32 P (measured 1.1e-3)
    assert errs[3] < 1e-4, errs
    assert errs[2] < 2e-3, errs
