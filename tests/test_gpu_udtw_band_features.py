"""The banded feature path (csrc/udtw_band.hip) for sequences of F >= 1 features.

With a Sakoe-Chiba band narrower than the grid, the cost max(S, 0) / var and
the penalty beta ln var are built only for the band's cells, in the band
layout that the banded sweep reads (one row of slots per anti-diagonal); the
backward sweep leaves dC / dQ in the same layout, and the gradients of X, Y
and the standard deviations are summed from it row by row and column by
column. Against the float64 oracle (its dense masked DP, udtw_cuda.cu:126-130):
distances, penalties and all four gradients, over one, two and four band
slots per lane, F below, at and above the reducer's 16-feature pass, F not a
multiple of 4, a single feature (D = 1, whose unbanded path builds the cost
in the sweep), fractional widths, the swapped orientation, soft-DTW (no
penalty) and float32 with R in double. Through the C ABI: the backward with
the forward's planes and with NULL (rebuilt) gives the same bits, and
variance inputs (sigma = 0) agree with standard deviations.
"""

import pytest
import torch

import torchwarp_amd as tw
from oracle import udtw as OU
from torchwarp_amd import _hip

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

f64, f32 = torch.float64, torch.float32


def _maxnorm(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


CASES = [  # (B, N, M, F, gamma, beta, bandwidth, dtype)
    (2, 300, 310, 16, 0.5, 1.0, 30.0, f64),      # one slot per lane
    (2, 290, 270, 4, 1.0, 1.0, 40.0, f64),       # N > M: the API swaps the sequences
    (1, 500, 500, 40, 0.7, 1.0, 80.0, f64),      # two slots; F > 16: reducer in passes
    (2, 250, 260, 3, 0.5, 0.0, 25.5, f64),       # soft-DTW, F odd, fractional width
    (1, 1000, 1000, 8, 1.0, 1.0, 130.0, f64),    # four slots per lane
    (2, 300, 310, 16, 0.5, 1.0, 30.0, f32),
    (1, 1024, 1024, 16, 0.1, 1.0, 102.0, f32),   # long and sharp: R in double
    (2, 300, 310, 1, 0.5, 1.0, 30.0, f64),       # D = 1
    (2, 290, 270, 1, 1.0, 1.0, 40.0, f64),       # D = 1, swapped
    (2, 250, 260, 1, 0.5, 0.0, 25.5, f64),       # D = 1 soft-DTW
    (1, 1024, 1024, 1, 0.1, 1.0, 102.0, f32),    # D = 1, R in double
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}N{}M{}F{}w{}{}{}".format(
    c[0], c[1], c[2], c[3], c[6], "" if c[5] else "-sdtw", "-f32" if c[7] == f32 else ""))
def test_banded_features_match_oracle(case):
    B, N, M, F, gamma, beta, band, dtype = case
    g = torch.Generator().manual_seed(N + F)
    X = torch.randn(B, N, F, generator=g, dtype=f64) / F ** 0.5
    Y = torch.randn(B, M, F, generator=g, dtype=f64) / F ** 0.5
    sx = 0.5 + torch.rand(B, N, 1, generator=g, dtype=f64)
    sy = 0.5 + torch.rand(B, M, 1, generator=g, dtype=f64)
    xs = [t.to("cuda", dtype).requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = tw.UDTW(gamma=gamma, beta=beta, bandwidth=band)(*xs)
    (d + 0.5 * p).sum().backward()
    ref = [t.clone().requires_grad_(True) for t in (X, Y, sx, sy)]
    rd, rp = OU.udtw(*ref, gamma=gamma, beta=beta, bandwidth=band)
    (rd + 0.5 * rp).sum().backward()
    got, want = [d, p] + [t.grad for t in xs], [rd, rp] + [t.grad for t in ref]
    if beta == 0.0:   # no penalty: the standard deviations get no gradient
        got, want = got[:1] + got[2:4], want[:1] + want[2:4]
    errs = [_maxnorm(a, b) for a, b in zip(got, want)]
    print("errors", errs)
    if dtype == f64:
        assert max(errs) < 1e-10, errs
    else:
        # gradients: 1.1e-3 is the float32 error of the unbanded path at
        # N = 1024, gamma = 0.1 with R in double
        assert max(errs[:2]) < 1e-5, errs
        assert max(errs[2:]) < 3e-3, errs


def _feat_fwd(X, Y, vx, vy, gamma, beta, band, sigma):
    dtype = X.dtype
    B, N, F = X.shape
    M = Y.shape[1]
    R = X.new_empty(B, _hip.carry_cols(N, M, gamma, dtype))
    P = X.new_empty(B, N * M)
    o1, o2 = X.new_empty(B), X.new_empty(B)
    nws = _hip.udtw_workspace_elems(B, N, M, F, dtype, band)
    ws = X.new_empty(nws)
    _hip.call("tw_udtw_feat_fwd", dtype, X, Y, vx, vy, B, N, M, F, gamma, beta, 1e-8, band,
              sigma, R, P, o1, o2, ws, nws * X.element_size())
    return R, P, o1, o2, ws


def _feat_bwd(X, Y, vx, vy, R, P, gr, gp, gamma, beta, band, sigma, fwd_ws):
    dtype = X.dtype
    B, N, F = X.shape
    M = Y.shape[1]
    nws = _hip.udtw_workspace_elems(B, N, M, F, dtype, band)
    grads = [torch.empty_like(t) for t in (X, Y, vx, vy)]
    _hip.call("tw_udtw_feat_bwd", dtype, X, Y, vx, vy, R, P, gr, gp, B, N, M, F, gamma, beta,
              1e-8, band, sigma, 1, *grads, fwd_ws, X.new_empty(nws), nws * X.element_size())
    return grads


def _inputs(B, N, M, F, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    X, Y = (torch.randn(B, L, F, generator=g, dtype=dtype).cuda() for L in (N, M))
    sx, sy = (0.5 + torch.rand(B, L, generator=g, dtype=dtype).cuda() for L in (N, M))
    gr, gp = (torch.rand(B, generator=g, dtype=dtype).cuda() for _ in range(2))
    return X, Y, sx, sy, gr, gp


@pytest.mark.parametrize("dtype", [f64, f32])
def test_backward_with_and_without_forward_planes(dtype):
    """The backward reads the band's cost from the forward's workspace, or
    rebuilds it when given NULL: the same bits either way."""
    B, N, M, F, gamma, beta, band = 3, 200, 210, 6, 0.7, 1.0, 20.0
    X, Y, sx, sy, gr, gp = _inputs(B, N, M, F, dtype, 12)
    R, P, _, _, ws = _feat_fwd(X, Y, sx, sy, gamma, beta, band, 1)
    outs = [_feat_bwd(X, Y, sx, sy, R, P, gr, gp, gamma, beta, band, 1, fw) for fw in (ws, None)]
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_variance_inputs_match_standard_deviations():
    """sigma = 0 takes variances v = s^2: the same distances, and variance
    gradients equal to the standard deviation's divided by 2 s."""
    B, N, M, F, gamma, beta, band = 2, 150, 160, 5, 0.5, 1.0, 15.0
    X, Y, sx, sy, gr, gp = _inputs(B, N, M, F, f64, 13)
    *fs, _ = _feat_fwd(X, Y, sx, sy, gamma, beta, band, 1)
    *fv, _ = _feat_fwd(X, Y, sx * sx, sy * sy, gamma, beta, band, 0)
    for a, b in zip(fs[2:], fv[2:]):
        assert _maxnorm(a, b) < 1e-13
    Rs, Ps, Rv, Pv = fs[0], fs[1], fv[0], fv[1]
    gs = _feat_bwd(X, Y, sx, sy, Rs, Ps, gr, gp, gamma, beta, band, 1, None)
    gv = _feat_bwd(X, Y, sx * sx, sy * sy, Rv, Pv, gr, gp, gamma, beta, band, 0, None)
    assert _maxnorm(gv[0], gs[0]) < 1e-12 and _maxnorm(gv[1], gs[1]) < 1e-12
    assert _maxnorm(gv[2], gs[2] / (2 * sx)) < 1e-12
    assert _maxnorm(gv[3], gs[3] / (2 * sy)) < 1e-12


def test_single_feature_band_takes_the_banded_path():
    """D = 1 with a band narrower than the grid runs banded: the forward needs
    the B*N*M-element plane (and the size query reports it), and its
    distances and gradients equal, to rounding, those of a D = 2 input whose
    second feature is zero (the builder and the reducer at F = 1 and 2)."""
    B, N, M, gamma, beta, band = 2, 300, 310, 0.5, 1.0, 30.0
    X, Y, sx, sy, gr, gp = _inputs(B, N, M, 1, f64, 14)
    assert _hip.udtw_workspace_elems(B, N, M, 1, f64, band) == B * N * M
    assert _hip.udtw_feat_plane(B, N, M, 1, f64, band)
    assert not _hip.udtw_feat_plane(B, N, M, 1, f64, 0.0)
    R = X.new_empty(B, _hip.carry_cols(N, M, gamma, f64))
    with pytest.raises(RuntimeError, match="workspace"):
        _hip.call("tw_udtw_feat_fwd", f64, X, Y, sx, sy, B, N, M, 1, gamma, beta, 1e-8, band, 1,
                  R, X.new_empty(B, N * M), X.new_empty(B), X.new_empty(B), None, 0)
    X2, Y2 = (torch.cat([t, torch.zeros_like(t)], dim=2) for t in (X, Y))
    outs = []
    for x, y in ((X, Y), (X2, Y2)):
        R, P, o1, o2, ws = _feat_fwd(x, y, sx, sy, gamma, beta, band, 1)
        g = _feat_bwd(x, y, sx, sy, R, P, gr, gp, gamma, beta, band, 1, ws)
        outs.append([o1, o2, g[0][..., :1], g[1][..., :1], g[2], g[3]])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert _maxnorm(a, b) < 1e-12
