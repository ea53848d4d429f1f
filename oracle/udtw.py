"""uDTW / soft-DTW oracle on CPU tensors (test infrastructure only).

Two independent restatements of the same recurrence are kept so that they
pin each other:

* ``dp_forward`` / ``dp_backward``: the analytic anti-diagonal form of the
  reference's portable backend (``udtw/_torch_dp.py:14-75``), with +inf
  borders, unreachable cells R = +inf / P = 0 and the Sakoe-Chiba mask. It is
  also the CPU baseline timed by ``bench.py``.
* ``dp_value``: an out-of-place, autograd-differentiable form with a large
  finite sentinel (the idea of ``udtw/_autograd.py:32-74``); torch autograd
  through it gives the gradients the analytic backward must reproduce.

Recurrence (uDTW, Wang & Koniusz ECCV 2022, as in ``udtw_cuda.cu:13-21``):

    R[i,j] = C[i,j] + softmin_g(R[i-1,j-1], R[i-1,j], R[i,j-1])
    P[i,j] = Q[i,j] + sum_k softmax(-R_k / g)_k P_k

Backward for L = gR * R[N-1,M-1] + gP * P[N-1,M-1], successors s of cell k:

    w      = exp((E_s - R_k) / g),   E_s = R_s - C_s
    Pbar_k = sum_s w Pbar_s
    Rbar_k = sum_s w (Rbar_s - Pbar_s (P_k - (P_s - Q_s)) / g)
    dL/dC = Rbar, dL/dQ = Pbar.
"""

import torch

INF = float("inf")
BIG = 1e20


def _rows(d, N, M):
    """Row indices i of anti-diagonal d (cells (i, d - i))."""
    return torch.arange(max(0, d - M + 1), min(N - 1, d) + 1)


# --------------------------------------------------------------- analytic form

def dp_forward(C, Q, gamma, bandwidth=0.0):
    """(R_end [B], P_end [B], R [B,N,M], P [B,N,M]); udtw/_torch_dp.py:14-42."""
    B, N, M = C.shape
    # one leading border row/column; the border is +inf except the origin
    R = C.new_full((B, N + 1, M + 1), INF)
    P = C.new_zeros((B, N + 1, M + 1))
    R[:, 0, 0] = 0.0
    for d in range(N + M - 1):
        i = _rows(d, N, M)
        j = d - i
        # padded coordinates of the three predecessors: diagonal, up, left
        pr = torch.stack((R[:, i, j], R[:, i, j + 1], R[:, i + 1, j]), dim=-1)
        pp = torch.stack((P[:, i, j], P[:, i, j + 1], P[:, i + 1, j]), dim=-1)
        z = -pr / gamma
        r = C[:, i, j] - gamma * torch.logsumexp(z, dim=-1)
        keep = torch.isfinite(r)
        if bandwidth > 0:
            keep = keep & ((i - j).abs() <= bandwidth)
        p = Q[:, i, j] + (torch.softmax(z, dim=-1) * pp).sum(-1)
        R[:, i + 1, j + 1] = torch.where(keep, r, INF)
        P[:, i + 1, j + 1] = torch.where(keep, p, 0.0)
    R, P = R[:, 1:, 1:], P[:, 1:, 1:]
    return R[:, -1, -1].clone(), P[:, -1, -1].clone(), R.contiguous(), P.contiguous()


def dp_backward(C, Q, R, P, grad_r, grad_p, gamma):
    """(dL/dC, dL/dQ), both [B,N,M]; udtw/_torch_dp.py:45-75."""
    B, N, M = C.shape
    # padded at the far end so successors never go out of range;
    # padding carries E = -inf (weight 0) and zero adjoints
    Gb = C.new_zeros((B, N + 1, M + 1))
    Hb = C.new_zeros((B, N + 1, M + 1))
    E = C.new_full((B, N + 1, M + 1), -INF)
    A = C.new_zeros((B, N + 1, M + 1))
    Gb[:, N - 1, M - 1] = grad_r
    Hb[:, N - 1, M - 1] = grad_p
    E[:, N - 1, M - 1] = R[:, -1, -1] - C[:, -1, -1]
    A[:, N - 1, M - 1] = P[:, -1, -1] - Q[:, -1, -1]
    for d in range(N + M - 3, -1, -1):
        i = _rows(d, N, M)
        j = d - i
        rk = R[:, i, j].unsqueeze(-1)
        pk = P[:, i, j].unsqueeze(-1)
        si = (i + 1, i, i + 1)
        sj = (j, j + 1, j + 1)
        Es = torch.stack([E[:, a, b] for a, b in zip(si, sj)], dim=-1)
        Gs = torch.stack([Gb[:, a, b] for a, b in zip(si, sj)], dim=-1)
        Hs = torch.stack([Hb[:, a, b] for a, b in zip(si, sj)], dim=-1)
        As = torch.stack([A[:, a, b] for a, b in zip(si, sj)], dim=-1)
        w = torch.exp((Es - rk) / gamma)
        Gb[:, i, j] = (w * (Gs - Hs * (pk - As) / gamma)).sum(-1)
        Hb[:, i, j] = (w * Hs).sum(-1)
        rk = rk.squeeze(-1)
        E[:, i, j] = torch.where(torch.isfinite(rk), rk - C[:, i, j], -INF)
        A[:, i, j] = pk.squeeze(-1) - Q[:, i, j]
    return Gb[:, :N, :M].contiguous(), Hb[:, :N, :M].contiguous()


# ----------------------------------------------------- costs from the features

def pairwise(X, Y, vx, vy, beta, eps):
    """(cost, penalty, sq_raw, var_raw) for X [B,N,D], Y [B,M,D], vx [B,N], vy [B,M].

    GEMM form of ||x - y||^2 as the reference builds it
    (udtw/_autograd.py:24-29): sq = max(x2 + y2 - 2 x.y, 0),
    var = max((vx + vy) / 2, eps), cost = sq / var, penalty = beta log var.
    """
    G = torch.bmm(X, Y.transpose(1, 2))
    x2 = (X * X).sum(-1)
    y2 = (Y * Y).sum(-1)
    sq_raw = x2.unsqueeze(2) + y2.unsqueeze(1) - 2.0 * G
    var_raw = 0.5 * (vx.unsqueeze(2) + vy.unsqueeze(1))
    sq, var = sq_raw.clamp_min(0), var_raw.clamp_min(eps)
    return sq / var, beta * torch.log(var), sq_raw, var_raw


def features_forward(X, Y, vx, vy, gamma, beta, eps, bandwidth=0.0):
    """uDTW from features: (distance [B], penalty [B], R, P)."""
    cost, pen, _, _ = pairwise(X, Y, vx, vy, beta, eps)
    return dp_forward(cost, pen, gamma, bandwidth)


def features_backward(X, Y, vx, vy, R, P, grad_r, grad_p, gamma, beta, eps):
    """(dX, dY, dvx, dvy); chain rule of udtw/_ops.py:200-211 and :179-183.

    Clamp gradients follow torch.clamp_min: zero where sq_raw <= 0 or
    var_raw <= eps.
    """
    cost, pen, sq_raw, var_raw = pairwise(X, Y, vx, vy, beta, eps)
    var = var_raw.clamp_min(eps)
    d_cost, d_pen = dp_backward(cost, pen, R, P, grad_r, grad_p, gamma)
    dsq = torch.where(sq_raw > 0, d_cost / var, 0.0)
    dvar = torch.where(var_raw > eps, (beta * d_pen - d_cost * cost) / var, 0.0)
    # sq = x2 + y2 - 2 G  =>  dX = -2 dsq Y + 2 X rowsum(dsq), likewise dY
    dX = -2.0 * torch.bmm(dsq, Y) + 2.0 * X * dsq.sum(2, keepdim=True)
    dY = -2.0 * torch.bmm(dsq.transpose(1, 2), X) + 2.0 * Y * dsq.sum(1).unsqueeze(-1)
    return dX, dY, 0.5 * dvar.sum(2), 0.5 * dvar.sum(1)


# ------------------------------------------------------- differentiable form

def dp_value(C, Q, gamma, bandwidth=0.0):
    """(distance [B], penalty [B]) built out of place, differentiable by autograd.

    Unreachable cells hold the finite sentinel BIG (value) and 0 (penalty).
    """
    B, N, M = C.shape
    rows = torch.arange(N)
    big1 = C.new_full((B, 1), BIG)
    zero1 = C.new_zeros((B, 1))
    R1 = R2 = C.new_full((B, N), BIG)   # diagonals d-1, d-2 indexed by row
    P1 = P2 = C.new_zeros((B, N))
    for d in range(N + M - 1):
        j = d - rows
        ok = (j >= 0) & (j < M)
        if bandwidth > 0:
            ok = ok & ((rows - j).abs() <= bandwidth)
        jj = j.clamp(0, M - 1)
        c, q = C[:, rows, jj], Q[:, rows, jj]
        if d == 0:
            r = torch.where(ok, c, BIG)
            p = torch.where(ok, q, 0.0)
        else:
            # row i of diagonal d: diag pred = row i-1 of d-2, up = row i-1 of
            # d-1, left = row i of d-1
            up_r = torch.cat((big1, R1[:, :-1]), 1)
            dg_r = torch.cat((big1, R2[:, :-1]), 1)
            up_p = torch.cat((zero1, P1[:, :-1]), 1)
            dg_p = torch.cat((zero1, P2[:, :-1]), 1)
            z = -torch.stack((dg_r, up_r, R1), -1) / gamma
            r = c - gamma * torch.logsumexp(z, -1)
            p = q + (torch.softmax(z, -1) * torch.stack((dg_p, up_p, P1), -1)).sum(-1)
            ok = ok & (r < 0.5 * BIG)
            r = torch.where(ok, r, BIG)
            p = torch.where(ok, p, 0.0)
        R2, R1, P2, P1 = R1, r, P1, p
    return R1[:, N - 1], P1[:, N - 1]


# ---------------------------------------------------------------- public API

def udtw_from_cost(cost, penalty, *, gamma=1.0, bandwidth=None):
    """Differentiable (distance, penalty); udtw/functional.py:104-144."""
    if cost.shape[1] > cost.shape[2]:
        cost, penalty = cost.transpose(1, 2), penalty.transpose(1, 2)
    return dp_value(cost, penalty, gamma, bandwidth or 0.0)


def udtw(X, Y, sigma_x, sigma_y, *, beta=1.0, gamma=1.0, normalize=False,
         bandwidth=None, eps=1e-8):
    """Differentiable uDTW (distance, penalty); udtw/functional.py:147-209."""
    def run(A, Bq, sa, sb):
        if A.shape[1] > Bq.shape[1]:      # the problem is symmetric; N <= M
            A, Bq, sa, sb = Bq, A, sb, sa
        cost, pen, _, _ = pairwise(A, Bq, sa.squeeze(-1) ** 2, sb.squeeze(-1) ** 2, beta, eps)
        return dp_value(cost, pen, gamma, bandwidth or 0.0)

    d, p = run(X, Y, sigma_x, sigma_y)
    if not normalize:
        return d, p
    dxx, pxx = run(X, X, sigma_x, sigma_x)
    dyy, pyy = run(Y, Y, sigma_y, sigma_y)
    return d - 0.5 * (dxx + dyy), p - 0.5 * (pxx + pyy)


def soft_dtw(X, Y, *, gamma=1.0, normalize=False, bandwidth=None):
    """soft-DTW = uDTW with sigma = 1, beta = 0 (sdtw.py:79-84)."""
    ox = X.new_ones(X.shape[0], X.shape[1], 1)
    oy = Y.new_ones(Y.shape[0], Y.shape[1], 1)
    d, _ = udtw(X, Y, ox, oy, beta=0.0, gamma=gamma, bandwidth=bandwidth)
    if not normalize:
        return d
    dxx, _ = udtw(X, X, ox, ox, beta=0.0, gamma=gamma, bandwidth=bandwidth)
    dyy, _ = udtw(Y, Y, oy, oy, beta=0.0, gamma=gamma, bandwidth=bandwidth)
    return d - 0.5 * (dxx + dyy)
