"""Autograd-native JEANIE / FVM / pairwise costs, used only for derivatives the
HIP kernels do not provide (forward mode and derivatives of a backward pass),
through torch.func on the inputs' own device -- as in the reference
(``jeanie/_autograd.py:1-74``). Finite sentinel BIG instead of +inf.
"""

import torch
import torch.nn.functional as F

BIG = 1e20


def _windows(x, s1, s2):
    nd = x.dim()
    return x.unfold(nd - 3, 2 * s1 + 1, 1).unfold(nd - 2, 2 * s2 + 1, 1)


def jeanie(cost, s1, s2, gamma):
    """cost [B,K1,K2,T,U] -> (distance [B], accumulator [B,K1,K2,T,U])."""
    B, K1, K2, T, U = cost.shape
    rows = torch.arange(T, device=cost.device)
    big_row = cost.new_full((B, K1, K2, T), BIG)
    big1 = cost.new_full((B, K1, K2, 1), BIG)
    diags = []
    R1 = R2 = big_row
    for d in range(T + U - 1):
        u = d - rows
        ok = (u >= 0) & (u < U)
        c = cost[..., rows, u.clamp(0, U - 1)]
        if d == 0:
            r = torch.where(ok, c, BIG)
        else:
            pr = torch.stack((torch.cat((big1, R1[..., :-1]), -1), R1,
                              torch.cat((big1, R2[..., :-1]), -1)), 0)
            pr = _windows(F.pad(pr, (0, 0, s2, s2, s1, s1), value=BIG), s1, s2)
            r = torch.where(ok, c - gamma * torch.logsumexp(-pr / gamma, dim=(0, 5, 6)), BIG)
        diags.append(r)
        R2, R1 = R1, r
    out = -gamma * torch.logsumexp(-R1[..., T - 1].reshape(B, -1) / gamma, dim=1)
    Rd = torch.stack(diags, -2)                      # [B,K1,K2,T+U-1,T]
    t = torch.arange(T, device=cost.device).view(T, 1)
    u = torch.arange(U, device=cost.device).view(1, U)
    return out, Rd[..., t + u, t]


def pair_cost(A, Bm, metric):
    """A [P,R,D], Bm [P,C,D] -> [P,R,C]; metric 0 raw, 1 squared, 2 Euclidean."""
    G = torch.bmm(A, Bm.transpose(1, 2))
    sq = (A * A).sum(-1, keepdim=True) + (Bm * Bm).sum(-1).unsqueeze(1) - 2.0 * G
    if metric == 0:
        return sq
    sq = sq.clamp_min(0)
    if metric == 1:
        return sq
    pos = sq > 0
    return torch.where(pos, torch.where(pos, sq, 1.0).sqrt(), 0.0)


def rbf_cost(A, Bm, sigma):
    """A [P,R,D], Bm [P,C,D] -> [P,R,C]: sum_d 2 - 2 exp(-sigma (a - b)^2)."""
    diff = A.unsqueeze(-2) - Bm.unsqueeze(-3)
    return (2.0 - 2.0 * torch.exp(-sigma * diff.pow(2))).sum(-1)


def cost_from_features(query, support, metric):
    B, K1, K2, T, D = query.shape
    cost = pair_cost(query.reshape(B, K1 * K2 * T, D), support, metric)
    return cost.view(B, K1, K2, T, support.shape[1])


def jeanie_features(query, support, s1, s2, gamma, metric):
    return jeanie(cost_from_features(query, support, metric), s1, s2, gamma)


def fvm(cost, gamma):
    """cost [B,K,T,U] -> distance [B] (viewpoint softmin, then soft-DTW)."""
    temporal = -gamma * torch.logsumexp(-cost / gamma, dim=1)
    return jeanie(temporal[:, None, None], 0, 0, gamma)[0]
