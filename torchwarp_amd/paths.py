"""Alignment paths (drop-in for ``torchwarp.paths``, ``src/torchwarp/paths.py:1-250``).

Each distance is a SoftMin_gamma over the path distances of all paths; for a
pair of sequences these functions return

* ``path_matrix``: the soft-selector-weighted path matrices, i.e. the
  gradient of the distance with respect to the cost, computed by the HIP
  backward kernels;
* ``optimal_path``: the path with the smallest distance (gamma = 0), from
  the float64 hard-DP kernel ``tw_optimal_path_f64``, whose indices are
  bitwise those of the reference's scan (``paths.py:85-127``).

Plotting (``torchwarp.plot``, matplotlib) is not part of this build.
"""

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import torch

from . import _hip
from .jeanie import euclidean_cost, fvm_from_cost, jeanie_from_cost, squared_euclidean_cost
from .sdtw import soft_dtw_from_cost
from .udtw import pairwise_matrices, udtw_from_cost

__all__ = ["Alignment", "soft_dtw", "soft_dtw_per_view", "udtw", "fvm", "jeanie", "optimal_path"]

_PLOTS = ("alignment", "path_3d", "twoway", "uncertainty")


@dataclass
class Alignment:
    """Result of a path computation (batched over the first dimension).

    Attributes:
        distance: [B] distance d.
        path_matrix: [B, T, U] (or [B, K, T, U]) soft-selector-weighted path matrices.
        optimal_path: per batch item, the cells (t, u) (or (t, u, k)) of the
            smallest-distance path from (0, 0) to (T-1, U-1).
        cost: the cost the paths are evaluated on (for uDTW: D * Sigma^dagger).
        Sigma: [B, T, U] pair-wise variances (uDTW only).
        Omega: [B] beta-weighted penalty (uDTW only).
        angles: viewpoint labels for the K axis, if given.
    """

    distance: torch.Tensor
    path_matrix: torch.Tensor
    optimal_path: List[List[Tuple[int, ...]]]
    cost: torch.Tensor
    Sigma: Optional[torch.Tensor] = None
    Omega: Optional[torch.Tensor] = None
    angles: Optional[list] = field(default=None)

    def plot(self, type="alignment", **kwargs):
        if type not in _PLOTS:
            raise ValueError("type must be one of {}".format(sorted(_PLOTS)))
        raise NotImplementedError("plotting (torchwarp.plot, matplotlib) is not part of "
                                  "torchwarp_amd")


def _value_and_grad(fn, D):
    """d = fn(D) and dd/dD (the path matrix)."""
    with torch.enable_grad():
        c = D.detach().clone().requires_grad_(True)
        d = fn(c)
        (g,) = torch.autograd.grad(d.sum(), c)
    return d.detach(), g.detach()


def _optimal(cost, max_shift, start_view):
    """cost [B, K, T, U] -> per item the list of (t, u, k) of the optimal path."""
    B, K, T, U = cost.shape
    c = cost.detach().to(torch.float64).contiguous()
    _hip.require(c, "auto", "optimal_path")
    if start_view is not None:
        sv = int(start_view)
        sv = sv + K if sv < 0 else sv   # numpy indexing, as the reference
        if not 0 <= sv < K:
            raise IndexError("start_view {} is out of bounds for {} viewpoints"
                             .format(start_view, K))
    else:
        sv = -1
    if B == 0:
        return []
    n = B * K * T * U
    r = c.new_empty(n)
    back = torch.empty(n, dtype=torch.int32, device=c.device)
    path = torch.empty(B, T + U - 1, 3, dtype=torch.int32, device=c.device)
    plen = torch.empty(B, dtype=torch.int32, device=c.device)
    _hip.call("tw_optimal_path", torch.float64, c, B, K, T, U, int(max_shift), sv, r, back, path,
              plen)
    path, plen = path.cpu().tolist(), plen.cpu().tolist()
    return [[tuple(cell) for cell in path[b][:plen[b]]] for b in range(B)]


def optimal_path(cost, *, max_shift=0, start_view=None):
    """Paths with the smallest distance for a batch of cost matrices.

    cost: [B, T, U] (cells (t, u)) or [B, K, T, U] (cells (t, u, k)).
    """
    if cost.ndim == 3:
        return [[(t, u) for t, u, _ in p] for p in _optimal(cost.unsqueeze(1), 0, None)]
    if cost.ndim != 4:
        raise ValueError("cost must have shape [B, T, U] or [B, K, T, U]")
    return _optimal(cost, max_shift, start_view)


def _base_distance(query, support, metric):
    if metric == "euclidean":
        return euclidean_cost(query, support)
    if metric == "sqeuclidean":
        return squared_euclidean_cost(query, support)
    raise ValueError("metric must be 'euclidean' or 'sqeuclidean'")


def soft_dtw(cost, *, gamma=0.1):
    """soft-DTW paths for a cost matrix [B, T, U]."""
    d, pm = _value_and_grad(lambda x: soft_dtw_from_cost(x, gamma=gamma), cost)
    return Alignment(d, pm, optimal_path(cost), cost)


def soft_dtw_per_view(query, support, *, gamma=0.1, metric="euclidean", angles=None):
    """soft-DTW of each query viewpoint separately; query [B, K, T, d], support [B, U, d].

    Returns a list of K Alignments with path cells (t, u, k).
    """
    D = _base_distance(query, support, metric)
    views = []
    for k in range(D.shape[1]):
        a = soft_dtw(D[:, k], gamma=gamma)
        a.optimal_path = [[(t, u, k) for t, u in p] for p in a.optimal_path]
        a.angles = angles
        views.append(a)
    return views


def udtw(X, Y, sigma_x, sigma_y, *, gamma=1.0, beta=1.0):
    """uDTW paths, evaluated on D * Sigma^dagger (uDTW Eq. 2); Sigma and the
    beta-weighted penalty Omega (Eq. 3) are returned alongside."""
    with torch.no_grad():
        DS, pen, Sigma = pairwise_matrices(X, Y, sigma_x, sigma_y, beta)
    d, pm = _value_and_grad(lambda x: udtw_from_cost(x, pen, gamma=gamma).distance, DS)
    with torch.no_grad():
        Omega = udtw_from_cost(DS, pen, gamma=gamma).penalty
    return Alignment(d, pm, optimal_path(DS), DS, Sigma=Sigma, Omega=Omega)


def fvm(query, support, *, gamma=0.1, metric="euclidean", angles=None):
    """FVM paths (free viewpoint at every step, JEANIE Eq. 13); query [B, K, T, d]."""
    D = _base_distance(query, support, metric)
    d, pm = _value_and_grad(lambda x: fvm_from_cost(x, gamma=gamma), D)
    return Alignment(d, pm, optimal_path(D, max_shift=D.shape[1]), D, angles=angles)


def jeanie(query, support, *, gamma=0.1, max_shift=1, metric="euclidean", angles=None,
           start_view=None):
    """JEANIE paths (one viewpoint axis); query [B, K, T, d], support [B, U, d].

    ``start_view`` restricts the paths to start at that viewpoint: the soft
    path matrix is computed with a 1e4 penalty on every other viewpoint's
    (0, 0) cell, the optimal path with the start restricted exactly.
    """
    D = _base_distance(query, support, metric)
    Ds = D
    if start_view is not None:
        penalty = torch.zeros_like(D)
        penalty[:, :, 0, 0] = 1e4
        penalty[:, start_view, 0, 0] = 0
        Ds = D + penalty
    d, pm = _value_and_grad(lambda x: jeanie_from_cost(x, gamma=gamma, max_shift=max_shift), Ds)
    return Alignment(d, pm, optimal_path(D, max_shift=max_shift, start_view=start_view), D,
                     angles=angles)
