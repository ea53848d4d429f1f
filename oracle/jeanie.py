"""JEANIE / FVM / soft-DTW-from-cost oracle on CPU tensors (test infrastructure only).

JEANIE (Wang et al., IJCV 2024, Algorithm 1 extended to two viewpoint axes),
as the reference's portable backend computes it (``jeanie/_torch_dp.py``):

    R[n,0,0] = C[n,0,0]
    R[n,t,u] = C[n,t,u] + softmin_g{ R[n',t',u'] : |n1'-n1| <= s1, |n2'-n2| <= s2,
                                      (t',u') in {(t-1,u), (t,u-1), (t-1,u-1)} }
    out      = softmin_g{ R[n,T-1,U-1] over all n }

Backward: Rbar_k = sum_s exp((E_s - R_k)/g) Rbar_s (+ dL/dR_k), E_s = R_s - C_s,
seeded with grad_out * softmax_n(-R[n,T-1,U-1]/g); dL/dC = Rbar.

``forward`` / ``backward`` restate ``jeanie/_torch_dp.py:14-75`` (inf-padded
viewpoint windows gathered with ``unfold``); ``value`` is an out-of-place
differentiable form with a finite sentinel (``jeanie/_autograd.py:20-55``).
"""

import torch
import torch.nn.functional as F

INF = float("inf")
BIG = 1e20


def _windows(x, s1, s2):
    """[..., K1+2s1, K2+2s2, L] -> [..., K1, K2, L, 2s1+1, 2s2+1] viewpoint windows."""
    nd = x.dim()
    return x.unfold(nd - 3, 2 * s1 + 1, 1).unfold(nd - 2, 2 * s2 + 1, 1)


def _rows(d, T, U):
    return torch.arange(max(0, d - U + 1), min(T - 1, d) + 1)


def forward(C, s1, s2, gamma):
    """C [B,K1,K2,T,U] -> (out [B], R [B,K1,K2,T,U]); jeanie/_torch_dp.py:14-42."""
    B, K1, K2, T, U = C.shape
    Rp = C.new_full((B, K1 + 2 * s1, K2 + 2 * s2, T + 1, U + 1), INF)
    a1, a2 = slice(s1, s1 + K1), slice(s2, s2 + K2)
    Rp[:, a1, a2, 1, 1] = C[..., 0, 0]
    for d in range(1, T + U - 1):
        t = _rows(d, T, U)
        u = d - t
        # padded temporal predecessors (t-1,u), (t,u-1), (t-1,u-1)
        pr = torch.stack((Rp[..., t, u + 1], Rp[..., t + 1, u], Rp[..., t, u]), 0)
        pr = _windows(pr, s1, s2)                      # [3,B,K1,K2,L,w1,w2]
        soft = -gamma * torch.logsumexp(-pr / gamma, dim=(0, 5, 6))
        Rp[:, a1, a2, t + 1, u + 1] = C[..., t, u] + soft
    R = Rp[:, a1, a2, 1:, 1:].contiguous()
    last = R[..., T - 1, U - 1].reshape(B, -1)
    return -gamma * torch.logsumexp(-last / gamma, dim=1), R


def backward(C, R, grad_out, s1, s2, gamma, grad_R=None):
    """dL/dC for L = sum_b grad_out[b] out[b] + <grad_R, R>; jeanie/_torch_dp.py:45-75."""
    B, K1, K2, T, U = C.shape
    shape = (B, K1 + 2 * s1, K2 + 2 * s2, T + 1, U + 1)
    Gp = C.new_zeros(shape)            # Rbar, padding 0
    Ep = C.new_full(shape, -INF)       # R - C, padding -inf (weight 0)
    a1, a2 = slice(s1, s1 + K1), slice(s2, s2 + K2)
    last = R[..., T - 1, U - 1]
    seed = grad_out.view(B, 1, 1) * torch.softmax(-last.reshape(B, -1) / gamma, 1).view(B, K1, K2)
    if grad_R is not None:
        seed = seed + grad_R[..., T - 1, U - 1]
    Gp[:, a1, a2, T - 1, U - 1] = seed
    Ep[:, a1, a2, T - 1, U - 1] = last - C[..., T - 1, U - 1]
    for d in range(T + U - 3, -1, -1):
        t = _rows(d, T, U)
        u = d - t
        succ = ((t + 1, u), (t, u + 1), (t + 1, u + 1))
        Es = _windows(torch.stack([Ep[..., a, b] for a, b in succ], 0), s1, s2)
        Gs = _windows(torch.stack([Gp[..., a, b] for a, b in succ], 0), s1, s2)
        rk = R[..., t, u]
        g = (torch.exp((Es - rk[None, ..., None, None]) / gamma) * Gs).sum(dim=(0, 5, 6))
        if grad_R is not None:
            g = g + grad_R[..., t, u]
        Gp[:, a1, a2, t, u] = g
        Ep[:, a1, a2, t, u] = rk - C[..., t, u]
    return Gp[:, a1, a2, :T, :U].contiguous()


def value(cost, s1, s2, gamma):
    """Differentiable (out [B], R [B,K1,K2,T,U]) with a finite sentinel."""
    B, K1, K2, T, U = cost.shape
    rows = torch.arange(T)
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
            pr = F.pad(pr, (0, 0, s2, s2, s1, s1), value=BIG)
            pr = _windows(pr, s1, s2)
            r = torch.where(ok, c - gamma * torch.logsumexp(-pr / gamma, dim=(0, 5, 6)), BIG)
        diags.append(r)
        R2, R1 = R1, r
    out = -gamma * torch.logsumexp(-R1[..., T - 1].reshape(B, -1) / gamma, dim=1)
    Rd = torch.stack(diags, -2)                      # [B,K1,K2,D,T]
    tt = torch.arange(T).view(T, 1)
    uu = torch.arange(U).view(1, U)
    return out, Rd[..., tt + uu, tt]


# ------------------------------------------------------------------ base costs

def _support(query, support):
    if support.ndim < 2 or query.ndim < support.ndim:
        raise ValueError("bad query/support ranks")
    return support.unsqueeze(-3) if query.ndim > support.ndim else support


def squared_euclidean_cost(query, support):
    """q2 + s2 - 2 q.s, clamped at 0 (jeanie/distances.py:25-31)."""
    s = _support(query, support)
    q2 = (query * query).sum(-1, keepdim=True)
    s2 = (s * s).sum(-1).unsqueeze(-2)
    return (q2 + s2 - 2.0 * torch.matmul(query, s.transpose(-1, -2))).clamp_min(0)


def euclidean_cost(query, support):
    """sqrt of the above with a zero gradient at zero distance (:34-38)."""
    sq = squared_euclidean_cost(query, support)
    pos = sq > 0
    return torch.where(pos, torch.where(pos, sq, 1.0).sqrt(), 0.0)


def rbf_cost(query, support, sigma=0.5):
    """sum_d 2 - 2 exp(-sigma (q_d - s_d)^2) (:41-51)."""
    s = _support(query, support)
    diff = query.unsqueeze(-2) - s.unsqueeze(-3)
    return (2.0 - 2.0 * torch.exp(-sigma * diff * diff)).sum(-1)


# ------------------------------------------------------------------ public API

def clamp_shifts(K1, K2, s1, s2):
    """Shifts beyond K-1 reach every viewpoint (jeanie/functional.py:48-50)."""
    return min(int(s1), K1 - 1), min(int(s2), K2 - 1)


def jeanie_from_cost(cost, *, gamma=0.1, max_shift=1, return_accumulator=False):
    """Differentiable; cost [B,K,T,U] (one axis) or [B,K1,K2,T,U]."""
    one = cost.ndim == 4
    c5 = cost.unsqueeze(2) if one else cost
    if isinstance(max_shift, int):
        sh = (max_shift, max_shift if not one else 0)
    else:
        sh = tuple(max_shift) + ((0,) if one else ())
    s1, s2 = clamp_shifts(c5.shape[1], c5.shape[2], *sh)
    T, U = c5.shape[3], c5.shape[4]
    tr = T > U
    out, R = value(c5.transpose(3, 4) if tr else c5, s1, s2, gamma)
    if tr:
        R = R.transpose(3, 4)
    if not return_accumulator:
        return out
    return out, (R[:, :, 0] if one else R)


def soft_dtw_from_cost(cost, *, gamma=1.0, bandwidth=None):
    """[B,T,U] -> [B]; sdtw.py:29-47."""
    if bandwidth:
        from .udtw import udtw_from_cost
        return udtw_from_cost(cost, torch.zeros_like(cost), gamma=gamma, bandwidth=bandwidth)[0]
    return jeanie_from_cost(cost[:, None], gamma=gamma, max_shift=0)


def fvm_from_cost(cost, *, gamma=0.1):
    """softmin over every viewpoint dim, then soft-DTW (jeanie/fvm.py:15-38)."""
    B, T, U = cost.shape[0], cost.shape[-2], cost.shape[-1]
    temporal = -gamma * torch.logsumexp(-cost.reshape(B, -1, T, U) / gamma, dim=1)
    return soft_dtw_from_cost(temporal, gamma=gamma)


def fvm_backward(cost, grad_out, gamma):
    """Analytic dL/dcost of fvm_from_cost for L = sum grad_out * d."""
    B, T, U = cost.shape[0], cost.shape[-2], cost.shape[-1]
    flat = cost.reshape(B, -1, T, U)
    temporal = -gamma * torch.logsumexp(-flat / gamma, dim=1)
    c5 = temporal[:, None, None]
    tr = T > U
    if tr:
        c5 = c5.transpose(3, 4)
    _, R = forward(c5, 0, 0, gamma)
    dt = backward(c5, R, grad_out, 0, 0, gamma)
    if tr:
        dt = dt.transpose(3, 4)
    w = torch.softmax(-flat / gamma, dim=1)
    return (w * dt[:, 0, 0].unsqueeze(1)).reshape(cost.shape)
