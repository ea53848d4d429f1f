"""uDTW functional interface (drop-in for ``torchwarp.udtw.functional``).

Same signatures, argument meaning and errors as the reference
(``src/torchwarp/udtw/functional.py:1-209``); the dynamic program runs on the
gfx950 HIP kernels through the custom ops of ``_ops``.

uDTW (Wang & Koniusz, ECCV 2022): uncertainty-weighted path cost (Eq. 2/16),
the uncertainty penalty under the same soft path distribution (Eq. 3), the
additive pairwise variance (Eq. 8) and the squared Euclidean base distance.
"""

from typing import NamedTuple

import torch

from .. import _hip
from . import _ops

_BACKENDS = ("auto", "cuda", "torch")


class UDTWOutput(NamedTuple):
    """Result of uDTW: ``distance`` [B] and the beta-weighted ``penalty`` [B]."""

    distance: torch.Tensor
    penalty: torch.Tensor


def _check_sequence_inputs(X, Y, sigma_x, sigma_y):
    if X.ndim != 3 or Y.ndim != 3:
        raise ValueError("X and Y must have shape [batch, time, feature]")
    if sigma_x.ndim != 3 or sigma_y.ndim != 3:
        raise ValueError("the uncertainties sigma must have shape [batch, time, 1]")
    if X.shape[0] != Y.shape[0]:
        raise ValueError("X and Y must have the same batch size")
    if X.shape[2] != Y.shape[2]:
        raise ValueError("X and Y must have the same feature dimension")
    if sigma_x.shape[:2] != X.shape[:2] or sigma_y.shape[:2] != Y.shape[:2]:
        raise ValueError("uncertainty tensors must match batch/time dimensions")
    if sigma_x.shape[2] != 1 or sigma_y.shape[2] != 1:
        raise ValueError("the uncertainties sigma must have shape [batch, time, 1]")
    if not X.is_floating_point() or not Y.is_floating_point():
        raise TypeError("X and Y must be floating-point tensors")
    if not sigma_x.is_floating_point() or not sigma_y.is_floating_point():
        raise TypeError("the uncertainties sigma must be floating-point tensors")


def _check_hyperparameters(gamma, beta, bandwidth):
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    if beta < 0:
        raise ValueError("beta must be >= 0")
    if bandwidth is not None and bandwidth < 0:
        raise ValueError("bandwidth must be None or >= 0")


def _squared_euclidean(X, Y, method="gemm"):
    """Pairwise squared distances [B,N,M]; "gemm" on the HIP pair-cost kernel,
    "diff" materialises x - y."""
    if method == "diff":
        return (X.unsqueeze(2) - Y.unsqueeze(1)).pow(2).sum(dim=3)
    if method != "gemm":
        raise ValueError("method must be 'gemm' or 'diff'")
    from ..jeanie.distances import squared_euclidean_cost
    return squared_euclidean_cost(X, Y)


def pairwise_matrices(X, Y, sigma_x, sigma_y, beta=1.0, eps=1e-8, *, method="gemm"):
    """Uncertainty-weighted cost, beta-weighted log-variance penalty, variance.

    Eq. (8):  Sigma_ij = 0.5 * (sigma_i^2 + sigma'_j^2)
    Eq. (16): cost_ij = ||x_i - y_j||^2 / Sigma_ij, penalty_ij = beta * log Sigma_ij
    """
    _check_sequence_inputs(X, Y, sigma_x, sigma_y)
    if eps <= 0:
        raise ValueError("eps must be > 0")
    if beta < 0:
        raise ValueError("beta must be >= 0")
    variance = (0.5 * (sigma_x.pow(2) + sigma_y.pow(2).transpose(1, 2))).clamp_min(eps)
    weighted_cost = _squared_euclidean(X, Y, method) / variance
    weighted_penalty = beta * torch.log(variance)
    return weighted_cost, weighted_penalty, variance


def _batchable(*tensors):
    """The normalized terms can run as one batch: equal lengths (dim 1), one
    dtype and one device, and a non-empty batch."""
    X = tensors[0]
    return (X.shape[0] > 0 and all(t.shape[1] == X.shape[1] for t in tensors)
            and all(t.dtype == X.dtype and t.device == X.device for t in tensors))


def _check_band_reached(band, N, M):
    """The reference raises when the distance is not finite under a band
    (udtw/functional.py:94-98). With finite costs that happens exactly when
    no monotone path stays within |i - j| <= band, i.e. |N - M| > band, so
    the check is made from the shapes: no device-to-host synchronisation,
    and banded calls capture in HIP graphs. (Non-finite inputs give a
    non-finite result instead of this error.)"""
    if band > 0 and abs(N - M) > band:
        raise ValueError("No valid DTW path reaches the final cell under the given bandwidth")


def udtw_from_cost(cost, penalty, *, gamma=1.0, bandwidth=None, backend="auto"):
    """Run the uDTW dynamic program on precomputed matrices.

    Args:
        cost: [B,N,M] uncertainty-weighted cost, e.g. D / Sigma.
        penalty: [B,N,M] per-cell penalty, e.g. beta * log Sigma.
        gamma: SoftMin temperature (> 0).
        bandwidth: Sakoe-Chiba band; None or 0 disables pruning.
        backend: "auto" or "cuda" (the HIP kernels); "torch" is not part of this build.

    Returns:
        UDTWOutput(distance [B], penalty [B]).
    """
    if cost.ndim != 3 or penalty.ndim != 3:
        raise ValueError("cost and penalty must have shape [B,N,M]")
    if cost.shape != penalty.shape:
        raise ValueError("cost and penalty must have identical shapes")
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    if bandwidth is not None and bandwidth < 0:
        raise ValueError("bandwidth must be None or >= 0")
    if backend not in _BACKENDS:
        raise ValueError("backend must be one of {}".format(_BACKENDS))
    if cost.shape[1] == 0 or cost.shape[2] == 0:
        raise ValueError("sequence lengths must be non-zero")
    if cost.dtype not in (torch.float32, torch.float64):
        cost, penalty = cost.float(), penalty.float()
    # the recurrence and the band are symmetric in (i, j): keep N <= M
    if cost.shape[1] > cost.shape[2]:
        cost = cost.transpose(1, 2)
        penalty = penalty.transpose(1, 2)
    band = 0.0 if bandwidth is None else float(bandwidth)
    _check_band_reached(band, cost.shape[1], cost.shape[2])
    distance, pen, _, _ = _ops.dp_apply(cost, penalty, float(gamma), band, backend)
    return UDTWOutput(distance, pen)


def _udtw_fused(X, Y, sigma_x, sigma_y, beta, gamma, bandwidth, eps, backend):
    """uDTW with the cost and penalty built inside the kernel (Eqs. 8, 16)."""
    if X.shape[1] > Y.shape[1]:  # symmetric problem; keep N <= M
        X, Y, sigma_x, sigma_y = Y, X, sigma_y, sigma_x
    dtype = X.dtype if X.dtype in (torch.float32, torch.float64) else torch.float32
    # the kernels square the standard deviations themselves (and return d sigma)
    X, Y, sx, sy = _hip.dense(dtype, X, Y, sigma_x, sigma_y, contiguous=False)
    if Y is X:
        # d(X, X): torch.compile cannot trace a Function receiving one tensor twice
        Y = X.view_as(X)
    if sy is sx:
        sy = sx.view_as(sx)
    band = 0.0 if bandwidth is None else float(bandwidth)
    _check_band_reached(band, X.shape[1], Y.shape[1])
    distance, pen, _, _, _ = _ops.fused_apply(X, Y, sx, sy, float(gamma), float(beta), float(eps),
                                           band, backend, True)
    return UDTWOutput(distance, pen)


def udtw(X, Y, sigma_x, sigma_y, *, beta=1.0, gamma=1.0, normalize=False, bandwidth=None,
         method="gemm", eps=1e-8, backend="auto"):
    """Uncertainty-DTW between two batches of sequences.

    Args:
        X, Y: [B,N,D], [B,M,D] sequences.
        sigma_x, sigma_y: [B,N,1], [B,M,1] positive standard deviations.
        beta: Penalty weight (>= 0).
        gamma: SoftMin temperature (> 0).
        normalize: If True, return d(X,Y) - 0.5 [d(X,X) + d(Y,Y)] for both
            the distance and the penalty.
        bandwidth: Sakoe-Chiba band; None or 0 disables pruning.
        method: "gemm" (cost built inside the fused kernel) or "diff"
            (materialised matrices, see ``pairwise_matrices``).
        eps: Lower bound applied to the variance.
        backend: "auto" or "cuda".

    Returns:
        UDTWOutput(distance [B], penalty [B]); the penalty is beta-weighted.
    """
    _check_sequence_inputs(X, Y, sigma_x, sigma_y)
    _check_hyperparameters(gamma, beta, bandwidth)
    if eps <= 0:
        raise ValueError("eps must be > 0")
    if method not in ("gemm", "diff"):
        raise ValueError("method must be 'gemm' or 'diff'")
    if backend not in _BACKENDS:
        raise ValueError("backend must be one of {}".format(_BACKENDS))
    if X.shape[1] == 0 or Y.shape[1] == 0:
        raise ValueError("sequence lengths must be non-zero")

    def run(A, Bq, sa, sb):
        if method == "gemm":
            return _udtw_fused(A, Bq, sa, sb, beta, gamma, bandwidth, eps, backend)
        cost, pen, _ = pairwise_matrices(A, Bq, sa, sb, beta, eps, method=method)
        return udtw_from_cost(cost, pen, gamma=gamma, bandwidth=bandwidth, backend=backend)

    if normalize and _batchable(X, Y, sigma_x, sigma_y):
        # d(X,Y), d(X,X) and d(Y,Y) share one grid shape when N == M: one
        # launch over 3B pairs (each pair is computed independently, so the
        # values are those of three separate calls)
        B = X.shape[0]
        d, p = run(torch.cat((X, X, Y)), torch.cat((Y, X, Y)),
                   torch.cat((sigma_x, sigma_x, sigma_y)), torch.cat((sigma_y, sigma_x, sigma_y)))
        (d_xy, d_xx, d_yy), (p_xy, p_xx, p_yy) = d.split(B), p.split(B)
        return UDTWOutput(d_xy - 0.5 * (d_xx + d_yy), p_xy - 0.5 * (p_xx + p_yy))
    d_xy, p_xy = run(X, Y, sigma_x, sigma_y)
    if not normalize:
        return UDTWOutput(d_xy, p_xy)
    d_xx, p_xx = run(X, X, sigma_x, sigma_x)
    d_yy, p_yy = run(Y, Y, sigma_y, sigma_y)
    return UDTWOutput(d_xy - 0.5 * (d_xx + d_yy), p_xy - 0.5 * (p_xx + p_yy))
