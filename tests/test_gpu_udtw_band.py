"""The banded sweep (csrc/udtw_band.hip) on precomputed matrices.

A Sakoe-Chiba band narrower than the grid runs a sweep over the band's cells
only, one wavefront per pair with lanes along the band, R / P stored
band-compressed. Distances, penalties and both gradients against the oracle
in float64 (1e-10) and float32, over band widths that take one, two and four
band slots per lane, both parities of the width, fractional widths, the
transposed orientation, soft-DTW (no penalty), float32 with R in double, and
gradients that must be exactly zero outside the band.
"""

import pytest
import torch

import torchwarp_amd.functional as TF
from oracle import udtw as OU

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

f64 = torch.float64


def _maxnorm(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


CASES = [  # (B, N, M, gamma, bandwidth, penalty, dtype)
    (3, 200, 210, 0.5, 20.0, True, f64),       # one slot per lane
    (2, 300, 300, 0.7, 37.0, True, f64),       # odd width
    (2, 400, 380, 0.5, 100.0, True, f64),      # two slots per lane, N > M
    (1, 600, 640, 1.0, 200.0, True, f64),      # four slots per lane
    (1, 1200, 1200, 1.0, 200.0, True, f64),    # banded, but 32 rows of 2w + 1
                                               # columns of both planes exceed
                                               # the LDS: no gather / scatter
    (2, 250, 260, 0.3, 12.5, True, f64),       # fractional width
    (2, 300, 320, 0.5, 24.0, False, f64),      # soft-DTW
    (2, 150, 170, 0.5, 20.0, True, f64),       # |N - M| = width
    (2, 300, 310, 1.0, 40.0, True, torch.float32),
    (1, 1024, 1024, 0.1, 102.0, True, torch.float32),   # R in double (long, sharp)
    (3, 500, 520, 1.0, 90.0, True, torch.float32),      # float, two slots per lane
    (2, 700, 700, 1.0, 180.0, True, torch.float32),     # float, four slots per lane
    (1, 900, 900, 0.5, 150.0, True, torch.float32),     # four slots, R in double
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}N{}M{}w{}{}{}".format(
    c[0], c[1], c[2], c[4], "" if c[5] else "-nopen", "-f32" if c[6] == torch.float32 else ""))
def test_banded_sweep_matches_oracle(case):
    B, N, M, gamma, band, pen, dtype = case
    g = torch.Generator().manual_seed(N + M)
    C = 3.0 * torch.rand(B, N, M, generator=g, dtype=f64)
    Q = 0.5 * torch.rand(B, N, M, generator=g, dtype=f64)
    wr = torch.rand(B, generator=g, dtype=f64) + 0.5
    wp = torch.rand(B, generator=g, dtype=f64) + 0.5
    c = C.to("cuda", dtype).requires_grad_(True)
    if pen:
        q = Q.to("cuda", dtype).requires_grad_(True)
        d, p = TF.udtw_from_cost(c, q, gamma=gamma, bandwidth=band)
        (d * wr.to("cuda", dtype) + p * wp.to("cuda", dtype)).sum().backward()
        rc, rq = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
        rd, rp = OU.udtw_from_cost(rc, rq, gamma=gamma, bandwidth=band)
        (rd * wr + rp * wp).sum().backward()
        got, want = [d, p, c.grad, q.grad], [rd, rp, rc.grad, rq.grad]
    else:
        d = TF.soft_dtw_from_cost(c, gamma=gamma, bandwidth=band)
        (d * wr.to("cuda", dtype)).sum().backward()
        rc = C.clone().requires_grad_(True)
        rd, _ = OU.udtw_from_cost(rc, torch.zeros_like(rc), gamma=gamma, bandwidth=band)
        (rd * wr).sum().backward()
        got, want = [d, c.grad], [rd, rc.grad]
    torch.cuda.synchronize()
    errs = [_maxnorm(a, b) for a, b in zip(got, want)]
    print(case, ["%.1e" % e for e in errs])
    if dtype == f64:
        assert max(errs) < 1e-10, errs
    else:
        assert max(errs[:len(errs) // 2]) < 1e-5 and max(errs) < 2e-3, errs
    # nothing outside the band
    i = torch.arange(N).view(-1, 1)
    j = torch.arange(M).view(1, -1)
    out = ((i - j).abs() > band).to("cuda")
    assert float(c.grad[:, out].abs().max()) == 0.0


@pytest.mark.parametrize("band,band_ws", [(20.0, False), (20.0, True), (0.0, False)],
                         ids=["banded", "banded-scatter", "general"])
@pytest.mark.parametrize("dtype", [torch.float32, f64], ids=["f32", "f64"])
def test_backward_with_gradients_at_odd_offsets(dtype, band, band_ws):
    """The cost-path backwards (the banded sweep, and the general sweep
    without a band) store the gradients in aligned pairs of row neighbours,
    chosen by the parity of each cell's address; with the band workspace the
    banded sweep keeps them in its band layout and a scatter pass writes them
    (the sweep's other workgroups zeroing the rest). Here d_cost starts at an
    odd element offset and d_pen at an even one, with N M odd (the pairs'
    parity alternates between batch entries), through the C ABI; against the
    oracle, and nothing outside the planes is written."""
    from torchwarp_amd import _hip
    B, N, M, gamma = 3, 151, 163, 0.5
    g = torch.Generator().manual_seed(7)
    C = 3.0 * torch.rand(B, N, M, generator=g, dtype=f64)
    Q = 0.5 * torch.rand(B, N, M, generator=g, dtype=f64)
    wr = torch.rand(B, generator=g, dtype=f64) + 0.5
    wp = torch.rand(B, generator=g, dtype=f64) + 0.5
    rc, rq = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    rd, rp = OU.udtw_from_cost(rc, rq, gamma=gamma, bandwidth=band or None)
    (rd * wr + rp * wp).sum().backward()

    dev = lambda t: t.to("cuda", dtype).contiguous()
    c, q = dev(C), dev(Q)
    R = torch.empty(B, _hip.carry_cols(N, M, gamma, dtype), device="cuda", dtype=dtype)
    P = torch.empty(B, N * M, device="cuda", dtype=dtype)
    d = torch.empty(B, device="cuda", dtype=dtype)
    p = torch.empty(B, device="cuda", dtype=dtype)
    _hip.call("tw_udtw_cost_fwd", dtype, c, q, B, N, M, gamma, band, R, P, d, p)
    n = B * N * M
    buf_c = torch.full((n + 3,), 7.0, device="cuda", dtype=dtype)
    buf_q = torch.full((n + 4,), 7.0, device="cuda", dtype=dtype)
    dc, dq = buf_c[1:1 + n], buf_q[2:2 + n]
    ws_n = _hip.udtw_cost_workspace_elems(B, N, M, dtype, band if band_ws else 0.0)
    if band_ws:
        assert ws_n > _hip.udtw_cost_workspace_elems(B, N, M, dtype)
    ws = torch.empty(max(ws_n, 1), device="cuda", dtype=dtype)
    _hip.call("tw_udtw_cost_bwd", dtype, c, q, R, P, dev(wr), dev(wp), B, N, M, gamma, band, 1,
              dc, dq, ws if ws_n else None, ws_n * ws.element_size())
    torch.cuda.synchronize()
    tol = 1e-10 if dtype == f64 else 2e-3
    assert _maxnorm(d, rd) < (1e-10 if dtype == f64 else 1e-5)
    assert _maxnorm(dc.view(B, N, M), rc.grad) < tol
    assert _maxnorm(dq.view(B, N, M), rq.grad) < tol
    # the elements around the planes are untouched
    assert float(buf_c[0]) == 7.0 and float(buf_c[-2]) == 7.0
    assert float(buf_q[1]) == 7.0 and float(buf_q[-2]) == 7.0
