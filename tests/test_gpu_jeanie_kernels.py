"""Every JEANIE DP kernel family against the float64 oracle, through the public API.

The launcher picks the kernel from the shape: the wavefront-per-pair kernels
(K <= 32 viewpoints, rows of up to 8 / 16 / 32 steps, 16 in float64, shifts
up to 2; with windows of one neighbour their padded-lane variants, which run
several wavefronts per pair for small batches), the workgroup-per-pair
kernels (K <= 64, shifts <= 2, longer rows) and the general ones (more
viewpoints or larger shifts). The shapes below put
each family (and each compiled row length) under the forward and the
backward, with one and two viewpoint axes, T > U (the transposed
orientation) and odd T (a half-empty last row pair).
"""

import pytest
import torch

from oracle import jeanie as OJ
import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

CASES = [  # (B, K1, K2, T, U, (s1, s2), gamma)
    (3, 1, 9, 5, 7, (0, 1), 0.1),      # one axis, rows of 8
    (4, 5, 5, 12, 16, (1, 1), 0.1),    # cfg5-like, rows of 16
    (2, 4, 6, 9, 6, (1, 1), 0.3),      # T > U: transposed plane, odd T
    (2, 3, 4, 7, 11, (2, 2), 0.2),     # shifts of 2 (window of 5)
    (2, 5, 5, 20, 30, (1, 1), 0.1),    # rows of 32 (float32) / beyond (float64)
    (2, 6, 6, 6, 9, (1, 1), 0.1),      # 36 viewpoints: workgroup-per-pair kernels
    (2, 2, 3, 10, 40, (1, 1), 0.1),    # rows of 40: workgroup-per-pair kernels
    (2, 9, 9, 5, 6, (1, 1), 0.1),      # 81 viewpoints: general kernels
    (2, 7, 1, 5, 8, (3, 0), 0.2),      # shift 3: general kernels
    # padded-lane windows (5 x 5 with shifts 1, or one axis with shift 1):
    # small batches run several wavefronts per pair (odd T: a half-empty row
    # pair), batches past half the SIMDs one wavefront per pair
    (3, 9, 1, 9, 8, (1, 0), 0.2),      # one axis, several wavefronts
    (600, 9, 1, 8, 8, (1, 0), 0.2),    # one axis, one wavefront per pair
    (600, 5, 5, 12, 16, (1, 1), 0.1),  # 5 x 5, one wavefront per pair
    # full rows (U equal to the compiled row length): dC in pairs of cells
    (2, 3, 4, 6, 16, (1, 1), 0.1),     # general wavefront kernel, stride-4 exchange
    (2, 2, 5, 7, 8, (2, 1), 0.2),      # general wavefront kernel, shift 2
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}K{}x{}T{}U{}s{}".format(*c[:6]))
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_jeanie_kernels_match_oracle(case, dtype):
    B, K1, K2, T, U, shift, gamma = case
    g = torch.Generator().manual_seed(7)
    c = 4 * torch.rand(B, K1, K2, T, U, generator=g, dtype=torch.float64)
    w = torch.rand(B, generator=g, dtype=torch.float64)
    x = c.to("cuda", dtype).requires_grad_(True)
    d = TF.jeanie_from_cost(x, gamma=gamma, max_shift=shift)
    (d * w.to("cuda", dtype)).sum().backward()
    s1, s2 = min(shift[0], K1 - 1), min(shift[1], K2 - 1)
    out, R = OJ.forward(c, s1, s2, gamma)
    dC = OJ.backward(c, R, w, s1, s2, gamma)
    for got, want, tol in ((d, out, 1e-5), (x.grad, dC, 2e-4)):
        got = got.detach().double().cpu()
        err = ((got - want).abs().max() / want.abs().max()).item()
        bound = 1e-10 if dtype == torch.float64 else tol
        assert err < bound, (case, dtype, err)
