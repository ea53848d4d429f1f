"""The reference's operator names and schemas, served by this build's kernels.

The reference registers ``torchwarp_udtw::{dp, dp_backward, fused,
fused_backward}`` (``udtw/_ops.py:100-211``) and ``torchwarp_jeanie::{dp,
dp_backward, features, features_backward}`` (``jeanie/_ops.py:110-230``).
Code, exported programs and compiled graphs that call them by name bind to
the operators below, which take the same arguments and return the same number
of tensors, each with a fake implementation, a vmap rule that folds the mapped
dimension into the batch and float32 autocast, as the reference's.

What the reference's forwards return for their backwards (R / P in its
diagonal-major layout, the Gram matrix G, the squared norms) is carried here
in this build's own form: R and P as this build's kernels keep them, the
squared-distance plane (uDTW, D > 1) or the cost plane (JEANIE) in G's place,
and empty tensors for the squared norms, which these kernels do not need.
These tensors are only meaningful as inputs of the matching backward, as in
the reference, where nothing else reads them. ``natural_R`` returns the JEANIE
accumulator R[B, K1, K2, T, U], as the reference's forward does.

The package's own autograd Functions call the private ``twamd_*`` operators
(``udtw/_ops.py``, ``jeanie/_ops.py``), which take the standard deviations
directly and return only what their backward reads.
"""

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _hip
from ._opsutil import register_autocast, register_vmap
from .jeanie import _ops as _jops
from .udtw import _ops as _uops

# ------------------------------------------------------------------- uDTW


@torch.library.custom_op("torchwarp_udtw::dp", mutates_args=())
def udtw_dp(cost: Tensor, penalty: Tensor, gamma: float, bandwidth: float,
            backend: str) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    out_r, out_p, R, P = _uops._dp_direct(cost, penalty, gamma, bandwidth, backend)
    return out_r, out_p, R, P


@udtw_dp.register_fake
def _(cost, penalty, gamma, bandwidth, backend):
    B, N, M = cost.shape
    P = cost.new_empty(B, N * M) if penalty.numel() else cost.new_empty(0)
    R = cost.new_empty(B, _hip.carry_cols(N, M, gamma, cost.dtype))
    return cost.new_empty(B), cost.new_empty(B), R, P


@torch.library.custom_op("torchwarp_udtw::dp_backward", mutates_args=())
def udtw_dp_backward(cost: Tensor, penalty: Tensor, R: Tensor, P: Tensor, grad_r: Tensor,
                     grad_p: Tensor, gamma: float, bandwidth: float,
                     backend: str) -> Tuple[Tensor, Tensor]:
    d_cost, d_pen = _uops._dp_backward_direct(cost, penalty, R, P, grad_r, grad_p, gamma,
                                              bandwidth, backend)
    return d_cost, d_pen


@udtw_dp_backward.register_fake
def _(cost, penalty, R, P, grad_r, grad_p, gamma, bandwidth, backend):
    return torch.empty_like(cost), (torch.empty_like(cost) if penalty.numel()
                                    else cost.new_empty(0))


@torch.library.custom_op("torchwarp_udtw::fused", mutates_args=())
def udtw_fused(X: Tensor, Y: Tensor, vx: Tensor, vy: Tensor, gamma: float, beta: float,
               eps: float, bandwidth: float, backend: str
               ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """vx, vy: variances [B, N] / [B, M] (as the reference's op takes them)."""
    out_r, out_p, R, P, S = _uops._fused_direct(X, Y, vx, vy, gamma, beta, eps, bandwidth,
                                                backend, False)
    return out_r, out_p, R, P, S, X.new_empty(0), X.new_empty(0)


@udtw_fused.register_fake
def _(X, Y, vx, vy, gamma, beta, eps, bandwidth, backend):
    B, N, M = X.shape[0], X.shape[1], Y.shape[1]
    P = X.new_empty(B, N * M) if beta != 0.0 else X.new_empty(0)
    S = _uops._feat_ws(X, N, M, bandwidth)
    R = X.new_empty(B, _hip.carry_cols(N, M, gamma, X.dtype))
    return X.new_empty(B), X.new_empty(B), R, P, S, X.new_empty(0), X.new_empty(0)


@torch.library.custom_op("torchwarp_udtw::fused_backward", mutates_args=())
def udtw_fused_backward(X: Tensor, Y: Tensor, vx: Tensor, vy: Tensor, R: Tensor, P: Tensor,
                        G: Tensor, x2: Tensor, y2: Tensor, grad_r: Tensor, grad_p: Tensor,
                        gamma: float, beta: float, eps: float, bandwidth: float, backend: str
                        ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Returns (dX, dY, dvx, dvy), dvx / dvy with respect to the variances.
    G is the forward's squared-distance plane (or empty: then recomputed)."""
    return _uops._fused_backward_direct(X, Y, vx, vy, R, P, G, grad_r, grad_p, gamma, beta, eps,
                                        bandwidth, backend, False)


@udtw_fused_backward.register_fake
def _(X, Y, vx, vy, R, P, G, x2, y2, grad_r, grad_p, gamma, beta, eps, bandwidth, backend):
    return torch.empty_like(X), torch.empty_like(Y), torch.empty_like(vx), torch.empty_like(vy)


# ----------------------------------------------------------------- JEANIE


@torch.library.custom_op("torchwarp_jeanie::dp", mutates_args=())
def jeanie_dp(cost: Tensor, s1: int, s2: int, gamma: float, backend: str,
              natural_R: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """Returns (out, R_d, R): R_d for the backward, R the accumulator when
    ``natural_R`` (else empty)."""
    out, R = _jops._dp_direct(cost, s1, s2, gamma, backend)
    return out, R, (R.clone() if natural_R else cost.new_empty(0))


@jeanie_dp.register_fake
def _(cost, s1, s2, gamma, backend, natural_R):
    return (cost.new_empty(cost.shape[0]), torch.empty_like(cost),
            torch.empty_like(cost) if natural_R else cost.new_empty(0))


@torch.library.custom_op("torchwarp_jeanie::dp_backward", mutates_args=())
def jeanie_dp_backward(cost: Tensor, R_d: Tensor, grad_out: Tensor, grad_R: Optional[Tensor],
                       s1: int, s2: int, gamma: float, backend: str) -> Tensor:
    return _jops._dp_backward_direct(cost, R_d, grad_out, grad_R, s1, s2, gamma, backend)


@jeanie_dp_backward.register_fake
def _(cost, R_d, grad_out, grad_R, s1, s2, gamma, backend):
    return torch.empty_like(cost)


# the reference's metric codes (jeanie/functional.py:16): 0 squared, 1 Euclidean
_REF_METRIC = {0: _hip.METRIC_SQEUC, 1: _hip.METRIC_EUC}


def _metric(metric):
    if metric not in _REF_METRIC:
        raise ValueError("metric must be 0 (squared Euclidean) or 1 (Euclidean)")
    return _REF_METRIC[metric]


@torch.library.custom_op("torchwarp_jeanie::features", mutates_args=())
def jeanie_features(query: Tensor, support: Tensor, s1: int, s2: int, gamma: float, metric: int,
                    backend: str, natural_R: bool
                    ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """metric: the reference's code, 0 squared Euclidean, 1 Euclidean.
    Returns (out, R_d, R, G, q_sq, s_sq): G is the cost plane the backward
    reads, q_sq / s_sq empty."""
    out, R, cost = _jops._features_direct(query, support, s1, s2, gamma, _metric(metric),
                                          backend)
    e = query.new_empty   # (outputs may not alias one another: a new empty tensor each)
    return out, R, (R.clone() if natural_R else e(0)), cost, e(0), e(0)


@jeanie_features.register_fake
def _(query, support, s1, s2, gamma, metric, backend, natural_R):
    B, K1, K2, T, _ = query.shape
    U = support.shape[1]
    plane = query.new_empty(B, K1, K2, T, U)
    return (query.new_empty(B), plane, torch.empty_like(plane) if natural_R else query.new_empty(0),
            torch.empty_like(plane), query.new_empty(0), query.new_empty(0))


@torch.library.custom_op("torchwarp_jeanie::features_backward", mutates_args=())
def jeanie_features_backward(query: Tensor, support: Tensor, R_d: Tensor, G: Tensor,
                             q_sq: Tensor, s_sq: Tensor, grad_out: Tensor,
                             grad_R: Optional[Tensor], s1: int, s2: int, gamma: float,
                             metric: int, backend: str) -> Tuple[Tensor, Tensor]:
    dq, ds = _jops._features_backward_direct(query, support, G, R_d, grad_out, grad_R, s1, s2,
                                             gamma, _metric(metric), backend)
    return dq, ds


@jeanie_features_backward.register_fake
def _(query, support, R_d, G, q_sq, s_sq, grad_out, grad_R, s1, s2, gamma, metric, backend):
    return torch.empty_like(query), torch.empty_like(support)


register_vmap(udtw_dp, 2)
register_vmap(udtw_dp_backward, 6)
register_vmap(udtw_fused, 4)
register_vmap(udtw_fused_backward, 11)
register_vmap(jeanie_dp, 1)
register_vmap(jeanie_dp_backward, 4)
register_vmap(jeanie_features, 2)
register_vmap(jeanie_features_backward, 8)
for _op in (udtw_dp, udtw_dp_backward, udtw_fused, udtw_fused_backward, jeanie_dp,
            jeanie_dp_backward, jeanie_features, jeanie_features_backward):
    register_autocast(_op)
