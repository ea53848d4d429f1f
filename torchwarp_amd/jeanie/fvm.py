"""Free Viewpoint Matching (FVM), Eq. (13) of the JEANIE paper (drop-in for
``torchwarp.jeanie.fvm``, fvm.py:1-67): a viewpoint SoftMin at every temporal
pair, then soft-DTW -- both inside the HIP FVM kernels.
"""

import math

import torch

from . import _ops
from .distances import euclidean_cost, rbf_cost, squared_euclidean_cost

_METRICS = {"euclidean": euclidean_cost, "sqeuclidean": squared_euclidean_cost,
            "rbf": rbf_cost}


def fvm_from_cost(cost, *, gamma=0.1, backend="auto"):
    """FVM on a precomputed cost [B, K..., T, U] (every dim between B and [T, U]
    is a viewpoint index reduced by SoftMin). Returns distance [B]."""
    if not cost.is_floating_point():
        raise TypeError("cost must be a floating-point tensor")
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    if cost.ndim < 4:
        raise ValueError("cost must be [B, K..., T, U] with at least one viewpoint dim")
    if backend not in ("auto", "cuda", "torch"):
        raise ValueError("backend must be one of ('auto', 'cuda', 'torch')")
    B, T, U = cost.shape[0], cost.shape[-2], cost.shape[-1]
    K = math.prod(cost.shape[1:-2])   # explicit, so an empty batch reshapes too
    flat = cost.reshape(B, K, T, U)
    if flat.dtype not in (torch.float32, torch.float64):
        flat = flat.float()
    out, _, _ = _ops.fvm_apply(flat, float(gamma), backend)
    return out


def fvm(query, support, *, gamma=0.1, metric="euclidean", backend="auto"):
    """FVM between viewpoint-augmented queries [B, K..., T, D] and supports
    [B, U, D] or [B, K'..., U, D]. Returns distance [B]."""
    if metric not in _METRICS:
        raise ValueError("metric must be one of {}".format(tuple(_METRICS)))
    if query.ndim < 4 or support.ndim < 3:
        raise ValueError("query must be [B, K..., T, D] and support [B, U, D] or "
                         "[B, K'..., U, D]")
    B, T, D = query.shape[0], query.shape[-2], query.shape[-1]
    U = support.shape[-2]
    q = query.reshape(B, math.prod(query.shape[1:-2]), T, D)
    if support.ndim == 3:
        cost = _METRICS[metric](q, support)
    else:
        s = support.reshape(B, math.prod(support.shape[1:-2]), U, D)
        cost = _METRICS[metric](q.unsqueeze(2), s.unsqueeze(1))
    return fvm_from_cost(cost, gamma=gamma, backend=backend)
