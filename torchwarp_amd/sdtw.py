"""soft-DTW (Cuturi & Blondel, ICML 2017); drop-in for ``torchwarp.sdtw`` (sdtw.py:1-136)."""

from typing import Optional

import torch
import torch.nn as nn

from .udtw import _ops as _udtw_ops
from .udtw.functional import _BACKENDS, _batchable, udtw, udtw_from_cost


def softmin(x: torch.Tensor, gamma: float, dim: Optional[int] = None) -> torch.Tensor:
    """Differentiable soft minimum -gamma * logsumexp(-x / gamma)."""
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    if dim is None:
        x = x.reshape(-1)
        dim = 0
    return -gamma * torch.logsumexp(-x / gamma, dim=dim)


def softmin_weights(values: torch.Tensor, gamma: float, dim: int = 0) -> torch.Tensor:
    """Weights of the soft minimum, softmax(-values / gamma) over ``dim``."""
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    return torch.softmax(-values / gamma, dim=dim)


def soft_dtw_from_cost(cost: torch.Tensor, *, gamma: float = 1.0,
                       bandwidth: Optional[float] = None, backend: str = "auto") -> torch.Tensor:
    """soft-DTW on a precomputed cost [B, T, U]; returns [B].

    The reference routes this through JEANIE with one viewpoint
    (sdtw.py:46); here it is the uDTW DP kernel with no penalty, which is
    the same recurrence.
    """
    if not cost.is_floating_point():
        raise TypeError("cost must be a floating-point tensor")
    if cost.ndim != 3:
        raise ValueError("cost must have shape [B, T, U]")
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    if backend not in _BACKENDS:
        raise ValueError("backend must be one of {}".format(_BACKENDS))
    if bandwidth:
        return udtw_from_cost(cost, torch.zeros_like(cost), gamma=gamma, bandwidth=bandwidth,
                              backend=backend).distance
    if cost.shape[1] == 0 or cost.shape[2] == 0:
        raise ValueError("cost dimensions must be non-empty")
    if cost.dtype not in (torch.float32, torch.float64):
        cost = cost.float()
    if cost.shape[1] > cost.shape[2]:
        cost = cost.transpose(1, 2)
    out, _, _, _ = _udtw_ops.dp_apply(cost, cost.new_empty(0), float(gamma), 0.0, backend)
    return out


def soft_dtw(X: torch.Tensor, Y: torch.Tensor, *, gamma: float = 1.0, normalize: bool = False,
             bandwidth: Optional[float] = None, dist_func=None,
             backend: str = "auto") -> torch.Tensor:
    """soft-DTW between batches X [B,N,D] and Y [B,M,D]; returns distance [B].

    normalize: the soft-DTW divergence d(X,Y) - 0.5 [d(X,X) + d(Y,Y)].
    dist_func: optional (X, Y) -> cost [B,N,M]; default squared Euclidean,
    built inside the kernel without storing the [B,N,M] matrix.
    """
    if gamma <= 0:
        raise ValueError("gamma must be > 0")
    if bandwidth is not None and bandwidth < 0:
        raise ValueError("bandwidth must be None or >= 0")
    if backend not in _BACKENDS:
        raise ValueError("backend must be one of {}".format(_BACKENDS))
    if X.ndim != 3 or Y.ndim != 3:
        raise ValueError("X and Y must have shape [batch, time, feature]")

    def run(A, B):
        if dist_func is None:
            # soft-DTW is uDTW with sigma = 1 (Sigma = 1) and beta = 0
            ones_a = A.new_ones(A.shape[0], A.shape[1], 1)
            ones_b = B.new_ones(B.shape[0], B.shape[1], 1)
            return udtw(A, B, ones_a, ones_b, beta=0.0, gamma=gamma, bandwidth=bandwidth,
                        backend=backend).distance
        cost = dist_func(A, B)
        return udtw_from_cost(cost, torch.zeros_like(cost), gamma=gamma, bandwidth=bandwidth,
                              backend=backend).distance

    if normalize and dist_func is None and _batchable(X, Y):
        # one launch over 3B pairs when N == M (see udtw; a user dist_func
        # keeps three calls, since it sees the whole batch)
        d_xy, d_xx, d_yy = run(torch.cat((X, X, Y)), torch.cat((Y, X, Y))).split(X.shape[0])
        return d_xy - 0.5 * (d_xx + d_yy)
    d = run(X, Y)
    if not normalize:
        return d
    return d - 0.5 * (run(X, X) + run(Y, Y))


class SoftDTW(nn.Module):
    """soft-DTW module; see ``soft_dtw``. Forward: X [B,N,D], Y [B,M,D] -> [B]."""

    def __init__(self, gamma=1.0, normalize=False, bandwidth=None, dist_func=None, *,
                 backend="auto"):
        super().__init__()
        if gamma <= 0:
            raise ValueError("gamma must be > 0")
        if bandwidth is not None and bandwidth < 0:
            raise ValueError("bandwidth must be None or >= 0")
        if backend not in _BACKENDS:
            raise ValueError("backend must be one of {}".format(_BACKENDS))
        self.gamma = float(gamma)
        self.normalize = bool(normalize)
        self.bandwidth = None if bandwidth is None else float(bandwidth)
        self.dist_func = dist_func
        self.backend = backend

    def forward(self, X, Y):
        return soft_dtw(X, Y, gamma=self.gamma, normalize=self.normalize,
                        bandwidth=self.bandwidth, dist_func=self.dist_func, backend=self.backend)

    def extra_repr(self):
        return "gamma={}, normalize={}, bandwidth={}, backend={!r}".format(
            self.gamma, self.normalize, self.bandwidth, self.backend)
