"""Hard (gamma = 0) alignment DP with backtrack (test infrastructure only).

Restates ``src/torchwarp/paths.py:85-127``: r[k,0,0] = D[k,0,0] (or only at
``start_view``); each cell takes the strict ``<`` minimum over predecessor
viewpoints kk ascending within the window, and for each kk the temporal
predecessors in the order (t-1,u-1), (t-1,u), (t,u-1); the path ends at the
first viewpoint attaining the minimum of r[:, T-1, U-1] (``np.argmin``).
The index output must be bit-exact, so the scan order is kept as is.
"""

import numpy as np


def optimal_3d(D, max_shift, start_view=None):
    """D: float64 ndarray [K, T, U] -> list of (t, u, k) from (0,0) to (T-1,U-1)."""
    K, T, U = D.shape
    r = np.full((K, T, U), np.inf)
    r[:, 0, 0] = D[:, 0, 0]
    if start_view is not None:
        r[:, 0, 0] = np.inf
        r[start_view, 0, 0] = D[start_view, 0, 0]
    back = np.zeros((K, T, U, 3), dtype=np.int64)
    for t in range(T):
        for u in range(U):
            if t == 0 and u == 0:
                continue
            for k in range(K):
                best, arg = np.inf, None
                for kk in range(max(0, k - max_shift), min(K, k + max_shift + 1)):
                    for a, b in ((t - 1, u - 1), (t - 1, u), (t, u - 1)):
                        if a >= 0 and b >= 0 and r[kk, a, b] < best:
                            best, arg = r[kk, a, b], (kk, a, b)
                if arg is not None:
                    r[k, t, u] = D[k, t, u] + best
                    back[k, t, u] = arg
    k, t, u = int(r[:, T - 1, U - 1].argmin()), T - 1, U - 1
    path = [(t, u, k)]
    while (t, u) != (0, 0):
        k, t, u = (int(v) for v in back[k, t, u])
        path.append((t, u, k))
    return path[::-1]


def optimal_path(cost, max_shift=0, start_view=None):
    """cost: [B,T,U] -> list of [(t,u)], or [B,K,T,U] -> list of [(t,u,k)]."""
    c = np.asarray(cost, dtype=np.float64)
    if c.ndim == 3:
        return [[(t, u) for t, u, _ in optimal_3d(x[None], 0)] for x in c]
    return [optimal_3d(x, max_shift, start_view) for x in c]
