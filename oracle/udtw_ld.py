"""uDTW in extended precision (numpy ``longdouble``) -- TEST INFRASTRUCTURE ONLY.

A third restatement of the uDTW forward, analytic backward and feature chain
rule (reference: ``src/torchwarp/udtw/_torch_dp.py:14-75``,
``src/torchwarp/udtw/_ops.py:179-183,200-211``,
``src/torchwarp/udtw/_autograd.py:24-29``), evaluated in the x86 80-bit
extended format (64-bit significand: 2^11 = 2048 times finer than float64).
It serves as the "truth" against which float64 results are judged where the
float64 rounding of the DP itself is the question: at gamma = 0.1 and
N = M = 1024 the accumulated cost reaches ~1e4, so every backward weight
exp((E_s - R_k) / gamma) is the exponential of a difference of two numbers
of that size, rounded to float64 first, in any float64 implementation.

Pinned in ``tests/test_oracle_longdouble.py`` against the float64 oracle on
small cases (where both are exact to ~1e-13) and against the brute-force
path enumeration.
"""

import numpy as np

LD = np.longdouble


def _lse_min(z, gamma):
    """-gamma * log(sum(exp(-z / gamma))) over the last axis, stably."""
    m = np.min(z, axis=-1, keepdims=True)
    fin = np.isfinite(m)
    mm = np.where(fin, m, LD(0))
    s = np.sum(np.exp(-(z - mm) / gamma), axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        out = mm - gamma * np.log(s)
    return np.where(fin, out, LD(np.inf))[..., 0]


def features_value_and_grads(X, Y, vx, vy, gamma, beta, eps=1e-8, grad_r=1.0, grad_p=1.0):
    """One pair: X [N, D], Y [M, D], variances vx [N], vy [M] (any float
    arrays, converted to longdouble). Returns (r, p, dX, dY, dvx, dvy) of
    L = grad_r * r + grad_p * p, all longdouble."""
    X, Y = np.asarray(X, LD), np.asarray(Y, LD)
    vx, vy = np.asarray(vx, LD), np.asarray(vy, LD)
    g, beta, eps = LD(gamma), LD(beta), LD(eps)
    N, M = X.shape[0], Y.shape[0]
    x2, y2 = (X * X).sum(1), (Y * Y).sum(1)
    sq_raw = x2[:, None] + y2[None, :] - 2 * (X @ Y.T)
    var_raw = (vx[:, None] + vy[None, :]) / 2
    sq, var = np.maximum(sq_raw, 0), np.maximum(var_raw, eps)
    C, Q = sq / var, beta * np.log(var)

    inf = LD(np.inf)
    R = np.full((N + 1, M + 1), inf, dtype=LD)
    P = np.zeros((N + 1, M + 1), dtype=LD)
    R[0, 0] = 0
    for d in range(N + M - 1):
        i = np.arange(max(0, d - M + 1), min(N - 1, d) + 1)
        j = d - i
        pr = np.stack((R[i, j], R[i, j + 1], R[i + 1, j]), -1)
        pp = np.stack((P[i, j], P[i, j + 1], P[i + 1, j]), -1)
        r = C[i, j] + _lse_min(pr, g)
        m = np.min(pr, -1, keepdims=True)
        w = np.exp(-(pr - m) / g)
        w = w / w.sum(-1, keepdims=True)
        R[i + 1, j + 1] = r
        P[i + 1, j + 1] = Q[i, j] + (w * pp).sum(-1)
    R, P = R[1:, 1:], P[1:, 1:]

    Gb = np.zeros((N + 1, M + 1), dtype=LD)
    Hb = np.zeros((N + 1, M + 1), dtype=LD)
    E = np.full((N + 1, M + 1), -inf, dtype=LD)
    A = np.zeros((N + 1, M + 1), dtype=LD)
    Gb[N - 1, M - 1], Hb[N - 1, M - 1] = LD(grad_r), LD(grad_p)
    E[N - 1, M - 1] = R[-1, -1] - C[-1, -1]
    A[N - 1, M - 1] = P[-1, -1] - Q[-1, -1]
    for d in range(N + M - 3, -1, -1):
        i = np.arange(max(0, d - M + 1), min(N - 1, d) + 1)
        j = d - i
        rk, pk = R[i, j][:, None], P[i, j][:, None]
        si, sj = (i + 1, i, i + 1), (j, j + 1, j + 1)
        Es = np.stack([E[a, b] for a, b in zip(si, sj)], -1)
        Gs = np.stack([Gb[a, b] for a, b in zip(si, sj)], -1)
        Hs = np.stack([Hb[a, b] for a, b in zip(si, sj)], -1)
        As = np.stack([A[a, b] for a, b in zip(si, sj)], -1)
        w = np.exp((Es - rk) / g)
        Gb[i, j] = (w * (Gs - Hs * (pk - As) / g)).sum(-1)
        Hb[i, j] = (w * Hs).sum(-1)
        E[i, j] = R[i, j] - C[i, j]
        A[i, j] = P[i, j] - Q[i, j]
    dC, dQ = Gb[:N, :M], Hb[:N, :M]

    dsq = np.where(sq_raw > 0, dC / var, LD(0))
    dvar = np.where(var_raw > eps, (beta * dQ - dC * C) / var, LD(0))
    dX = -2 * (dsq @ Y) + 2 * X * dsq.sum(1)[:, None]
    dY = -2 * (dsq.T @ X) + 2 * Y * dsq.sum(0)[:, None]
    return R[-1, -1], P[-1, -1], dX, dY, dvar.sum(1) / 2, dvar.sum(0) / 2
