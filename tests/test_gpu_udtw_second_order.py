"""Second-order uDTW / soft-DTW / FVM through the public API, and the HIP
second-order entry points.

The double backward and forward-over-reverse of ``udtw_from_cost``, of
``udtw`` from features and of ``fvm_from_cost`` are checked against double
autograd through the oracle's differentiable DP on the CPU.

``tw_udtw_cost_tangent_*`` (the HIP tangent sweeps) are switched off: their
first GPU run stopped with a memory aperture violation whose cause was not
found (the same sweeps run on the CPU under AddressSanitizer, with every
index in bounds and results equal to the oracle's, in
``tests/test_tangent_host.py``). The entry points now refuse to launch, which
is tested here; their parity test against ``oracle/udtw_tangent.py`` is kept,
skipped, for when they are switched back on.
"""

import pytest
import torch

import torchwarp_amd.functional as TF
from torchwarp_amd import _hip

from oracle import udtw as OU
from oracle.udtw_tangent import dp_tangent as oracle_tangent

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

f64 = torch.float64


def _rand(shape, seed, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return shift + scale * torch.rand(shape, generator=g, dtype=f64)


def _rel(got, want):
    den = want.abs().max().item()
    return (got.double().cpu() - want).abs().max().item() / (den if den > 0 else 1.0)


CASES = [  # (B, N, M, gamma, bandwidth, penalty, dtype)
    (3, 5, 7, 0.7, 0.0, True, f64),
    (2, 6, 6, 0.4, 2.0, True, f64),
    (2, 9, 5, 0.5, 0.0, True, f64),          # N > M: any orientation
    (4, 140, 140, 1.0, 0.0, True, f64),      # the forecasting batch's pair shape
    (2, 140, 150, 1.0, 0.0, False, f64),     # soft-DTW: no penalty
    (2, 100, 120, 0.3, 15.0, True, f64),     # band
    (1, 600, 650, 1.0, 0.0, True, f64),      # more rows than threads: row loop
    (1, 900, 920, 2.0, 0.0, True, f64),      # exchanged diagonals past the LDS
    (2, 140, 140, 1.0, 0.0, True, torch.float32),
    (2, 300, 310, 1.0, 30.0, False, torch.float32),
]


def _case_inputs(B, N, M, seed):
    C = _rand((B, N, M), seed, 3.0)
    Q = _rand((B, N, M), seed + 1, 0.5)
    tC = _rand((B, N, M), seed + 2, 2.0, -1.0)
    tQ = _rand((B, N, M), seed + 3, 2.0, -1.0)
    g = [_rand((B,), seed + 4 + k, 2.0, -1.0) for k in range(4)]
    return C, Q, tC, tQ, g


def _tangent(C, Q, tC, tQ, gr, gp, tgr, tgp, gamma, band, pen, dtype):
    """tw_udtw_cost_tangent_* through the C ABI (device tensors)."""
    dev = lambda t: t.to("cuda", dtype).contiguous()
    B, N, M = C.shape
    out_c, out_q = torch.empty_like(dev(C)), torch.empty_like(dev(C))
    t_r, t_p = torch.empty(B, device="cuda", dtype=dtype), torch.zeros(B, device="cuda",
                                                                      dtype=dtype)
    nws = _hip.udtw_tangent_workspace_elems(B, N, M, pen, dtype)
    ws = torch.empty(nws, device="cuda", dtype=dtype)
    _hip.call("tw_udtw_cost_tangent", dtype, dev(C), dev(Q) if pen else None, dev(tC),
              dev(tQ) if pen else None, dev(gr), dev(gp) if pen else None, dev(tgr),
              dev(tgp) if pen else None, B, N, M, gamma, band, out_c, out_q if pen else None,
              t_r, t_p if pen else None, ws, ws.numel() * ws.element_size())
    return out_c, out_q, t_r, t_p


@pytest.mark.skip(reason="tw_udtw_cost_tangent_* are switched off: their first GPU run stopped "
                         "with a memory aperture violation whose cause is not yet found")
@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}N{}M{}w{}{}{}".format(
    c[0], c[1], c[2], c[4], "" if c[5] else "-nopen", "-f32" if c[6] == torch.float32 else ""))
def test_tangent_entry_point_matches_oracle(case):
    B, N, M, gamma, band, pen, dtype = case
    C, Q, tC, tQ, (gr, gp, tgr, tgp) = _case_inputs(B, N, M, seed=N + M)
    if not pen:
        Q, tQ, gp, tgp = (torch.zeros_like(t) for t in (Q, tQ, gp, tgp))
    want = oracle_tangent(C, Q, tC, tQ, gr, gp, tgr, tgp, gamma, band)
    got = _tangent(C, Q, tC, tQ, gr, gp, tgr, tgp, gamma, band, pen, dtype)
    torch.cuda.synchronize()
    tol = 1e-10 if dtype == f64 else 2e-4
    for k in ((0, 1, 2, 3) if pen else (0, 2)):
        assert _rel(got[k], want[k]) < tol, (k, _rel(got[k], want[k]))


def test_tangent_entry_point_refuses_to_launch():
    """Switched off: the arguments are still checked, then the call returns
    an error without launching anything."""
    C, Q, tC, tQ, (gr, gp, tgr, tgp) = _case_inputs(2, 6, 7, seed=1)
    with pytest.raises(RuntimeError, match="disabled"):
        _tangent(C, Q, tC, tQ, gr, gp, tgr, tgp, 0.5, 0.0, True, f64)
    with pytest.raises(RuntimeError, match="workspace"):
        _hip.call("tw_udtw_cost_tangent", f64, C.cuda(), None, None, None, gr.cuda(), None,
                  None, None, 2, 6, 7, 1.0, 0.0, torch.empty_like(C.cuda()), None, None, None,
                  None, 0)
    torch.cuda.synchronize()


def _double_autograd_cost(C, Q, vC, vQ, a, b, gamma, band):
    """HVP of L = a r + b p through the oracle's differentiable DP (CPU)."""
    C, Q = C.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    r, p = OU.dp_value(C, Q, gamma, band)
    dC, dQ = torch.autograd.grad((a * r + b * p).sum(), (C, Q), create_graph=True)
    return torch.autograd.grad((dC * vC).sum() + (dQ * vQ).sum(), (C, Q))


@pytest.mark.parametrize("band", [None, 6.0])
def test_double_backward_of_udtw_from_cost(band):
    B, N, M, gamma = 3, 40, 45, 0.5
    C, Q = _rand((B, N, M), 31, 3.0), _rand((B, N, M), 32, 0.5)
    vC, vQ = _rand((B, N, M), 33, 2.0, -1.0), _rand((B, N, M), 34, 2.0, -1.0)
    a, b = torch.tensor([1.0, 0.5, -2.0], dtype=f64), torch.tensor([0.3, 1.0, 2.0], dtype=f64)
    want = _double_autograd_cost(C, Q, vC, vQ, a, b, gamma, band or 0.0)
    c, q = C.cuda().requires_grad_(True), Q.cuda().requires_grad_(True)
    d, p = TF.udtw_from_cost(c, q, gamma=gamma, bandwidth=band)
    dC, dQ = torch.autograd.grad((a.cuda() * d + b.cuda() * p).sum(), (c, q), create_graph=True)
    hC, hQ = torch.autograd.grad((dC * vC.cuda()).sum() + (dQ * vQ.cuda()).sum(), (c, q))
    assert _rel(hC, want[0]) < 1e-10 and _rel(hQ, want[1]) < 1e-10


def test_forward_over_reverse_of_udtw_from_cost():
    B, N, M, gamma = 2, 30, 33, 0.7
    C, Q = _rand((B, N, M), 41, 3.0), _rand((B, N, M), 42, 0.5)
    vC = _rand((B, N, M), 43, 2.0, -1.0)
    want = _double_autograd_cost(C, Q, vC, torch.zeros_like(Q), torch.ones(B, dtype=f64),
                                 torch.ones(B, dtype=f64), gamma, 0.0)[0]
    _, hv = torch.func.jvp(lambda c: torch.func.grad(
        lambda x: sum(t.sum() for t in TF.udtw_from_cost(x, Q.cuda(), gamma=gamma)))(c),
        (C.cuda(),), (vC.cuda(),))
    assert _rel(hv, want) < 1e-10


def test_double_backward_of_udtw_from_features():
    """Feature path: PyTorch cost planes composed with the HIP DP; against
    double autograd through the oracle's features and DP on the CPU."""
    B, N, M, D, gamma, beta = 2, 20, 24, 3, 0.6, 0.8
    g = torch.Generator().manual_seed(51)
    X, Y = torch.randn(B, N, D, generator=g, dtype=f64), torch.randn(B, M, D, generator=g, dtype=f64)
    SX = 0.5 + torch.rand(B, N, 1, generator=g, dtype=f64)
    SY = 0.5 + torch.rand(B, M, 1, generator=g, dtype=f64)
    V = torch.randn(B, N, D, generator=g, dtype=f64)

    def loss_cpu(x):
        C, Qm, _, _ = OU.pairwise(x, Y, SX[..., 0] ** 2, SY[..., 0] ** 2, beta, 1e-8)
        r, p = OU.dp_value(C, Qm, gamma)
        return (r + 2.0 * p).sum()
    x = X.clone().requires_grad_(True)
    gx, = torch.autograd.grad(loss_cpu(x), x, create_graph=True)
    want, = torch.autograd.grad((gx * V).sum(), x)

    xg = X.cuda().requires_grad_(True)
    d, p = TF.udtw(xg, Y.cuda(), SX.cuda(), SY.cuda(), gamma=gamma, beta=beta)
    gx2, = torch.autograd.grad((d + 2.0 * p).sum(), xg, create_graph=True)
    got, = torch.autograd.grad((gx2 * V.cuda()).sum(), xg)
    assert _rel(got, want) < 1e-9, _rel(got, want)


def test_double_backward_of_fvm_from_cost():
    B, K, T, U, gamma = 2, 3, 12, 10, 0.4
    cost = _rand((B, K, T, U), 61, 2.0)
    V = _rand((B, K, T, U), 62, 2.0, -1.0)

    def fvm_cpu(c):
        temporal = -gamma * torch.logsumexp(-c / gamma, dim=1)
        return OU.dp_value(temporal, torch.zeros_like(temporal), gamma)[0]
    c = cost.clone().requires_grad_(True)
    gc, = torch.autograd.grad(fvm_cpu(c).sum(), c, create_graph=True)
    want, = torch.autograd.grad((gc * V).sum(), c)
    cg = cost.cuda().requires_grad_(True)
    gc2, = torch.autograd.grad(TF.fvm_from_cost(cg, gamma=gamma).sum(), cg, create_graph=True)
    got, = torch.autograd.grad((gc2 * V.cuda()).sum(), cg)
    assert _rel(got, want) < 1e-10, _rel(got, want)
