"""Second-order uDTW / soft-DTW oracle on CPU tensors (test infrastructure only).

The reference differentiates through its first-order backward by running
torch.func over an autograd-native restatement of the dynamic program
(``udtw/_ops.py:322-327`` ``DPBackward.backward``, ``udtw/_ops.py:329-339``
``DPBackward.jvp``, on ``udtw/_autograd.py:32-74``). What that computes, for
L = gR * r + gP * p with r = R[N-1,M-1], p = P[N-1,M-1] (the recurrences of
``oracle/udtw.py``), is the derivative of the first-order gradient

    (dL/dC, dL/dQ) = (Gt, At)

along a direction (tC, tQ, tgR, tgP). It is restated here as two explicit
tangent recursions, the form the HIP kernels implement:

forward tangent, cell (i,j) with predecessors k, softmin weights w_k:

    tR   = tC + sum_k w_k tR_k                       (tRbar = tR - tC)
    tw_k = -(w_k / g) (tR_k - tRbar)
    tP   = tQ + sum_k (w_k tP_k + tw_k P_k)          (tPbar = tP - tQ)

backward tangent, cell k with successors s (w = exp((Rbar_s - R_k)/g),
tw = -(w/g)(tR_k - tRbar_s), dP = P_k - Pbar_s, tdP = tP_k - tPbar_s):

    At_k  = sum_s w At_s
    tAt_k = sum_s (w tAt_s + tw At_s)
    Gt_k  = sum_s (w Gt_s - w At_s dP / g)
    tGt_k = sum_s (w tGt_s + tw Gt_s - (w tAt_s + tw At_s) dP / g - w At_s tdP / g)

with Gt = gR, At = gP, tGt = tgR, tAt = tgP at the end cell. The outputs are
(tGt, tAt) -- the tangent of (dL/dC, dL/dQ) -- and (tR, tP) at the end cell,
the tangents of r and p. Since (dL/dC, dL/dQ) is the gradient of L, its
Jacobian in (C, Q) is L's (symmetric) Hessian, so with tgR = tgP = 0 the same
numbers are the vector-Jacobian product a double backward needs, and (tR, tP)
at the end are its gradients with respect to gR and gP.

Unreachable cells (+inf R, and those outside the Sakoe-Chiba band) carry zero
tangents and zero weight.
"""

import torch

INF = float("inf")


def _rows(d, N, M):
    return torch.arange(max(0, d - M + 1), min(N - 1, d) + 1)


def dp_tangent(C, Q, tC, tQ, grad_r, grad_p, t_grad_r, t_grad_p, gamma, bandwidth=0.0):
    """(tGt [B,N,M], tAt [B,N,M], t_r [B], t_p [B]) for the recursions above.

    C, Q, tC, tQ: [B,N,M]; grad_r, grad_p, t_grad_r, t_grad_p: [B].
    """
    B, N, M = C.shape
    g = float(gamma)
    # one border row/column in front (forward) and behind (backward)
    R = C.new_full((B, N + 1, M + 1), INF)
    P = C.new_zeros((B, N + 1, M + 1))
    tR = C.new_zeros((B, N + 1, M + 1))
    tP = C.new_zeros((B, N + 1, M + 1))
    R[:, 0, 0] = 0.0
    for d in range(N + M - 1):
        i = _rows(d, N, M)
        j = d - i
        pr = torch.stack((R[:, i, j], R[:, i, j + 1], R[:, i + 1, j]), -1)
        pp = torch.stack((P[:, i, j], P[:, i, j + 1], P[:, i + 1, j]), -1)
        tr = torch.stack((tR[:, i, j], tR[:, i, j + 1], tR[:, i + 1, j]), -1)
        tp = torch.stack((tP[:, i, j], tP[:, i, j + 1], tP[:, i + 1, j]), -1)
        w = torch.softmax(-pr / g, -1)
        w = torch.where(torch.isfinite(pr), w, 0.0)
        r = C[:, i, j] - g * torch.logsumexp(-pr / g, -1)
        keep = torch.isfinite(r)
        if bandwidth > 0:
            keep = keep & ((i - j).abs() <= bandwidth)
        pbar = (w * pp).sum(-1)
        trbar = (w * tr).sum(-1)
        tw = -(w / g) * (tr - trbar.unsqueeze(-1))
        tpbar = (w * tp + tw * pp).sum(-1)
        R[:, i + 1, j + 1] = torch.where(keep, r, INF)
        P[:, i + 1, j + 1] = torch.where(keep, Q[:, i, j] + pbar, 0.0)
        tR[:, i + 1, j + 1] = torch.where(keep, tC[:, i, j] + trbar, 0.0)
        tP[:, i + 1, j + 1] = torch.where(keep, tQ[:, i, j] + tpbar, 0.0)
    R, P, tR, tP = (t[:, 1:, 1:] for t in (R, P, tR, tP))

    # backward: padded behind so that successors never leave the array; the
    # padding holds Rbar = -inf (weight 0) and zero adjoints
    def plane(fill):
        return C.new_full((B, N + 1, M + 1), fill)
    Rb, Pb, tRb, tPb = plane(-INF), plane(0.0), plane(0.0), plane(0.0)
    Gt, At, tGt, tAt = plane(0.0), plane(0.0), plane(0.0), plane(0.0)

    def store_bars(i, j):
        r = R[:, i, j]
        Rb[:, i, j] = torch.where(torch.isfinite(r), r - C[:, i, j], -INF)
        Pb[:, i, j] = P[:, i, j] - Q[:, i, j]
        tRb[:, i, j] = tR[:, i, j] - tC[:, i, j]
        tPb[:, i, j] = tP[:, i, j] - tQ[:, i, j]

    last_i, last_j = torch.tensor([N - 1]), torch.tensor([M - 1])
    reach = torch.isfinite(R[:, -1, -1])
    Gt[:, N - 1, M - 1] = torch.where(reach, grad_r, 0.0)
    At[:, N - 1, M - 1] = torch.where(reach, grad_p, 0.0)
    tGt[:, N - 1, M - 1] = torch.where(reach, t_grad_r, 0.0)
    tAt[:, N - 1, M - 1] = torch.where(reach, t_grad_p, 0.0)
    store_bars(last_i, last_j)
    for d in range(N + M - 3, -1, -1):
        i = _rows(d, N, M)
        j = d - i
        si, sj = (i + 1, i, i + 1), (j, j + 1, j + 1)

        def succ(t):
            return torch.stack([t[:, a, b] for a, b in zip(si, sj)], -1)
        rk = R[:, i, j].unsqueeze(-1)
        ok = torch.isfinite(rk)
        w = torch.where(ok, torch.exp((succ(Rb) - torch.where(ok, rk, 0.0)) / g), 0.0)
        tw = -(w / g) * (tR[:, i, j].unsqueeze(-1) - succ(tRb))
        dP = P[:, i, j].unsqueeze(-1) - succ(Pb)
        tdP = tP[:, i, j].unsqueeze(-1) - succ(tPb)
        As, tAs, Gs, tGs = succ(At), succ(tAt), succ(Gt), succ(tGt)
        At[:, i, j] = (w * As).sum(-1)
        tAt[:, i, j] = (w * tAs + tw * As).sum(-1)
        Gt[:, i, j] = (w * Gs - w * As * dP / g).sum(-1)
        tGt[:, i, j] = (w * tGs + tw * Gs - (w * tAs + tw * As) * dP / g
                        - w * As * tdP / g).sum(-1)
        store_bars(i, j)
    return (tGt[:, :N, :M].contiguous(), tAt[:, :N, :M].contiguous(),
            tR[:, -1, -1].clone(), tP[:, -1, -1].clone())
