"""Autograd-native uDTW, used only for derivatives the HIP kernels do not provide.

First-order reverse mode always runs the HIP backward kernel. Forward mode
(jvp) and differentiating *through* that backward (create_graph=True, MAML,
torch.func.hessian, ...) re-derive the derivative from this out-of-place
formulation with torch.func, on the inputs' own device -- the design of the
reference (``udtw/_autograd.py:1-79``). Unreachable cells carry the finite
sentinel BIG instead of +inf so that no derivative of logsumexp/softmax is NaN.
"""

import torch

BIG = 1e20


def matrices_from_features(X, Y, vx, vy, beta, eps):
    """Eqs. (8), (16) with the GEMM form of ||x - y||^2."""
    G = torch.bmm(X, Y.transpose(1, 2))
    x2, y2 = (X * X).sum(-1), (Y * Y).sum(-1)
    sq = (x2.unsqueeze(2) + y2.unsqueeze(1) - 2.0 * G).clamp_min(0)
    var = (0.5 * (vx.unsqueeze(2) + vy.unsqueeze(1))).clamp_min(eps)
    return sq / var, beta * torch.log(var)


def udtw(cost, penalty, gamma, bandwidth):
    """(distance [B], penalty [B]) for [B,N,M] matrices, differentiable to any order."""
    B, N, M = cost.shape
    rows = torch.arange(N, device=cost.device)
    big1 = cost.new_full((B, 1), BIG)
    zero1 = cost.new_zeros((B, 1))
    R1 = R2 = cost.new_full((B, N), BIG)
    P1 = P2 = cost.new_zeros((B, N))
    for d in range(N + M - 1):
        j = d - rows
        ok = (j >= 0) & (j < M)
        if bandwidth > 0:
            ok = ok & ((rows - j).abs() <= bandwidth)
        jj = j.clamp(0, M - 1)
        c, q = cost[:, rows, jj], penalty[:, rows, jj]
        if d == 0:
            r = torch.where(ok, c, BIG)
            p = torch.where(ok, q, 0.0)
        else:
            z = -torch.stack((torch.cat((big1, R2[:, :-1]), 1),
                              torch.cat((big1, R1[:, :-1]), 1), R1), -1) / gamma
            pp = torch.stack((torch.cat((zero1, P2[:, :-1]), 1),
                              torch.cat((zero1, P1[:, :-1]), 1), P1), -1)
            r = c - gamma * torch.logsumexp(z, -1)
            p = q + (torch.softmax(z, -1) * pp).sum(-1)
            ok = ok & (r < 0.5 * BIG)
            r = torch.where(ok, r, BIG)
            p = torch.where(ok, p, 0.0)
        R2, R1, P2, P1 = R1, r, P1, p
    return R1[:, N - 1], P1[:, N - 1]


def udtw_features(X, Y, vx, vy, gamma, beta, eps, bandwidth):
    cost, pen = matrices_from_features(X, Y, vx, vy, beta, eps)
    return udtw(cost, pen, gamma, bandwidth)
