"""Batched base distances (drop-in for ``torchwarp.jeanie.distances``, distances.py:1-51).

Two layouts, as in the reference:
  JEANIE / FVM:  query [..., K, T, D], support [..., U, D] -> [..., K, T, U]
  two sequences: x [..., N, D], y [..., M, D] (same rank) -> [..., N, M]

The (squared) Euclidean costs run on the HIP pair-cost kernel (matrix cores
for float32), the RBF cost on its own HIP kernel: batch dimensions where the
support broadcasts over the query are folded into the rows of one pairwise
block, so the support is never expanded in memory.
"""

import math

import torch

from . import _ops


def _check(query, support):
    if support.ndim < 2 or query.ndim < support.ndim:
        raise ValueError("query must be [..., K, T, D] or [..., N, D] and support "
                         "[..., U, D] or [..., M, D]")
    if query.shape[-1] != support.shape[-1]:
        raise ValueError("query/support feature dimensions do not match")
    # JEANIE layout: broadcast the support over the viewpoint dim of the query
    return support.unsqueeze(-3) if query.ndim > support.ndim else support


def _pair_cost(query, support, metric=None, sigma=None):
    s = _check(query, support)
    dtype = torch.promote_types(query.dtype, s.dtype)
    if dtype not in (torch.float32, torch.float64):
        dtype = torch.float32
    q, s = query.to(dtype), s.to(dtype)
    T, D, U = q.shape[-2], q.shape[-1], s.shape[-2]
    batch = torch.broadcast_shapes(q.shape[:-2], s.shape[:-2])
    sb = (1,) * (len(batch) - (s.ndim - 2)) + tuple(s.shape[:-2])
    f = len(batch)
    while f > 0 and sb[f - 1] == 1:      # trailing dims the support broadcasts over
        f -= 1
    lead, fold = batch[:f], batch[f:]
    P, F = math.prod(lead), math.prod(fold)
    A = q.expand(*batch, T, D).reshape(P, F * T, D)
    Bm = s.expand(*lead, *sb[f:], U, D).reshape(P, U, D)
    if sigma is None:
        cost = _ops.pair_apply(A, Bm, metric, "auto")
    else:
        cost = _ops.rbf_apply(A, Bm, float(sigma), "auto")
    return cost.reshape(*batch, T, U)


def squared_euclidean_cost(query: torch.Tensor, support: torch.Tensor) -> torch.Tensor:
    """Squared-Euclidean base distance."""
    return _pair_cost(query, support, _ops.METRIC_CODES["sqeuclidean"])


def euclidean_cost(query: torch.Tensor, support: torch.Tensor) -> torch.Tensor:
    """Euclidean base distance; the gradient at zero distance is 0."""
    return _pair_cost(query, support, _ops.METRIC_CODES["euclidean"])


def rbf_cost(query: torch.Tensor, support: torch.Tensor, sigma: float = 0.5) -> torch.Tensor:
    """RBF-style base cost d(x,y) = sum_d [2 - 2 exp(-sigma (x_d - y_d)^2)].

    This per-dimension form is not a matrix product. The HIP kernel sums the
    terms per output cell; the reference's [..., K, T, U, D] difference
    tensor is never formed.
    """
    if sigma <= 0:
        raise ValueError("sigma must be > 0")
    return _pair_cost(query, support, sigma=sigma)
