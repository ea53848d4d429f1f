"""Brute-force enumeration of every monotone alignment path (tiny sizes only).

Pins the DP restatements independently of the recurrence: the soft distance
is softmin_g over path sums, its gradient with respect to the cost is the
softmax-weighted path-indicator matrix, and gamma = 0 picks the argmin path.
Same enumeration as the reference's own test (``tests/test_paths.py:99-132``),
written here from the definition of a JEANIE path: steps (1,0), (0,1), (1,1)
in (t, u) and a viewpoint change of at most ``max_shift`` per step, starting
at any viewpoint.
"""

import itertools

import torch


def all_paths(K, T, U, max_shift):
    """Every path as a list of (t, u, k) cells from (0,0,*) to (T-1,U-1,*)."""
    out = []

    def walk(t, u, k, acc):
        if (t, u) == (T - 1, U - 1):
            out.append(acc)
            return
        for dt, du in ((1, 0), (0, 1), (1, 1)):
            if t + dt >= T or u + du >= U:
                continue
            for dk in range(-max_shift, max_shift + 1):
                if 0 <= k + dk < K:
                    walk(t + dt, u + du, k + dk, acc + [(t + dt, u + du, k + dk)])

    for k in range(K):
        walk(0, 0, k, [(0, 0, k)])
    return out


def soft_value_and_grad(cost, gamma, max_shift):
    """cost [K, T, U] float64 -> (softmin of path sums, path-probability matrix)."""
    K, T, U = cost.shape
    paths = all_paths(K, T, U, max_shift)
    w = torch.stack([sum(cost[k, t, u] for t, u, k in p) for p in paths])
    prob = torch.softmax(-w / gamma, 0)
    pm = torch.zeros_like(cost)
    for a, p in zip(prob, paths):
        for t, u, k in p:
            pm[k, t, u] += a
    return -gamma * torch.logsumexp(-w / gamma, 0), pm, paths, w


def udtw_value(cost, pen, gamma):
    """Brute force uDTW on one [N, M] pair: (softmin of path costs,
    softmax-weighted mean of path penalties)."""
    N, M = cost.shape
    paths = all_paths(1, N, M, 0)
    w = torch.stack([sum(cost[t, u] for t, u, _ in p) for p in paths])
    q = torch.stack([sum(pen[t, u] for t, u, _ in p) for p in paths])
    prob = torch.softmax(-w / gamma, 0)
    return -gamma * torch.logsumexp(-w / gamma, 0), (prob * q).sum()


def exact_dtw(cost):
    """Hard DTW on [T, U] by the textbook recursion."""
    T, U = cost.shape
    R = [[float("inf")] * (U + 1) for _ in range(T + 1)]
    R[0][0] = 0.0
    for t, u in itertools.product(range(1, T + 1), range(1, U + 1)):
        R[t][u] = float(cost[t - 1, u - 1]) + min(R[t - 1][u], R[t][u - 1], R[t - 1][u - 1])
    return R[T][U]
