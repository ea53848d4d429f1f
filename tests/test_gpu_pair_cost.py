"""Pairwise cost kernels (matrix-core forward, fused / FMA backward) against a
float64 evaluation of the same formulas.

Reference formulas (jeanie/distances.py:25-38, udtw/_autograd.py:24-29):
S = |a|^2 + |b|^2 - 2 a.b, squared-Euclidean max(S, 0), Euclidean
sqrt(max(S, 0)) with zero gradient at zero distance. The check runs on ragged
shapes that exercise partial 16-row / 16-column tiles, D that is and is not a
multiple of 4 and 16 (the float32 matrix-core forward takes 16-byte chunks or
single elements; float64 runs the FMA forward), D on both sides of the
matrix-core backward's limit of 64, and C on both sides of the fused
backward's limit. float64 within 1e-10 and float32 within 1e-5 of the
largest entry (values and gradients; random inputs keep every distance clear
of zero, where the GEMM form cancels).
"""

import pytest
import torch

import torchwarp_amd as tw

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

SHAPES = [  # (P, R, C, D)
    (3, 37, 5, 20),
    (2, 16, 48, 12),
    (1, 70, 33, 4),
    (2, 9, 8, 7),
    (4, 72, 8, 256),
    (1, 40, 80, 16),
    # more than 64 columns: the tiled backward passes, ragged tiles
    (2, 130, 70, 5),
    (1, 65, 129, 33),
    (2, 200, 100, 64),
    (3, 100, 90, 3),
    (1, 30, 200, 75),   # D > 64 and not a multiple of 4: backward by feature slices
    (2, 80, 90, 128),   # two whole 64-feature slices
]


def _ref(A, Bm, metric):
    A, Bm = A.double(), Bm.double()
    S = (A * A).sum(-1, keepdim=True) + (Bm * Bm).sum(-1).unsqueeze(1) - 2 * A @ Bm.transpose(1, 2)
    c = S.clamp_min(0)
    return c.sqrt() if metric == "euclidean" else c


def _maxnorm(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean"])
@pytest.mark.parametrize("shape", SHAPES)
def test_pair_cost_matches_float64(shape, metric, dtype):
    P, R, C, D = shape
    g = torch.Generator().manual_seed(P * 1000 + R * 10 + C + D)
    A = torch.randn(P, R, D, generator=g, dtype=torch.float64)
    Bm = torch.randn(P, C, D, generator=g, dtype=torch.float64)
    W = torch.randn(P, R, C, generator=g, dtype=torch.float64)
    fn = tw.euclidean_cost if metric == "euclidean" else tw.squared_euclidean_cost

    a = A.to("cuda", dtype).requires_grad_(True)
    b = Bm.to("cuda", dtype).requires_grad_(True)
    got = fn(a, b)
    (got * W.to("cuda", dtype)).sum().backward()

    # reference gradients from the float64 closed form on the same rounded inputs
    ra = A.to(dtype).double().requires_grad_(True)
    rb = Bm.to(dtype).double().requires_grad_(True)
    want = _ref(ra, rb, metric)
    S = want if metric == "sqeuclidean" else want ** 2
    dS = W * (S > 0)
    if metric == "euclidean":
        dS = torch.where(want > 0, 0.5 * W / want.clamp_min(1e-300), torch.zeros_like(W))
    da = 2 * (dS.sum(2, keepdim=True) * ra - dS @ rb)
    db = 2 * (dS.sum(1).unsqueeze(-1) * rb - dS.transpose(1, 2) @ ra)

    tol = 1e-10 if dtype == torch.float64 else 1e-5
    assert _maxnorm(got, want) < tol
    assert _maxnorm(a.grad, da) < tol
    assert _maxnorm(b.grad, db) < tol


RBF_SHAPES = [  # (query shape, support shape, sigma)
    ((3, 5, 8), (3, 6, 8), 0.5),          # two sequences
    ((2, 4, 7, 16), (2, 9, 16), 0.3),     # JEANIE layout: support broadcast over K
    ((2, 9, 8, 256), (2, 8, 256), 0.5),   # cfg4-like features
    ((1, 33, 3), (1, 70, 3), 2.0),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shapes", RBF_SHAPES, ids=lambda s: "x".join(map(str, s[0])))
def test_rbf_cost_matches_oracle(shapes, dtype):
    """HIP RBF cost (jeanie/distances.py:41-51) against the float64 oracle, which
    forms the reference's difference tensor; values and both gradients."""
    from oracle import jeanie as OJ
    qs, ss, sigma = shapes
    g = torch.Generator().manual_seed(9)
    q = torch.randn(*qs, generator=g, dtype=torch.float64) * 0.7
    s = torch.randn(*ss, generator=g, dtype=torch.float64) * 0.7
    w = torch.rand(*OJ.rbf_cost(q, s, sigma).shape, generator=g, dtype=torch.float64)
    a, b = q.to("cuda", dtype).requires_grad_(True), s.to("cuda", dtype).requires_grad_(True)
    out = tw.rbf_cost(a, b, sigma=sigma)
    (out * w.to("cuda", dtype)).sum().backward()
    rq, rs = q.clone().requires_grad_(True), s.clone().requires_grad_(True)
    ref = OJ.rbf_cost(rq, rs, sigma)
    (ref * w).sum().backward()
    tol = 1e-10 if dtype == torch.float64 else 1e-5
    assert out.dtype == dtype and out.shape == ref.shape
    assert _maxnorm(out, ref) < tol
    assert _maxnorm(a.grad, rq.grad) < tol
    assert _maxnorm(b.grad, rs.grad) < tol


def test_rbf_cost_vmap_and_autocast():
    """The RBF op under vmap (folded into the pair dimension) and autocast
    (computed in float32, as registered)."""
    g = torch.Generator().manual_seed(13)
    q = torch.randn(3, 2, 4, 5, 6, generator=g, dtype=torch.float64).cuda()
    s = torch.randn(3, 2, 7, 6, generator=g, dtype=torch.float64).cuda()
    got = torch.func.vmap(lambda a, b: tw.rbf_cost(a, b, sigma=0.4))(q, s)
    want = torch.stack([tw.rbf_cost(q[i], s[i], sigma=0.4) for i in range(3)])
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    with torch.autocast("cuda", dtype=torch.float16):
        half = tw.rbf_cost(q[0].half(), s[0].half(), sigma=0.4)
    assert half.dtype == torch.float32
    torch.testing.assert_close(half.double(), tw.rbf_cost(q[0].half().double(),
                                                          s[0].half().double(), sigma=0.4),
                               rtol=1e-5, atol=1e-5)
