"""uDTW / soft-DTW as PyTorch custom operators over the HIP kernels, plus autograd Functions.

Operator contract of the reference (``udtw/_ops.py:1-458``): ``custom_op``
kernels with fake implementations, vmap rules and float32 autocast, wrapped in
``autograd.Function``s (``setup_context`` style, ``generate_vmap_rule``,
``jvp``) so torch.compile, torch.func and create_graph=True all work.

* ``twamd_udtw::dp`` / ``dp_backward``: DP on precomputed cost / penalty
  (reference ops ``torchwarp_udtw::dp`` / ``dp_backward``, :100-138).
  An empty penalty tensor means "no penalty" (soft-DTW).
* ``twamd_udtw::fused`` / ``fused_backward``: DP straight from the features,
  the cost built inside the kernel (``torchwarp_udtw::fused`` /
  ``fused_backward``, :157-211). No Gram matrix and no layout permutation is
  materialised on the host side.

R and P are internal [B, N*M] tensors carried from forward to backward
(``R`` scaled by log2(e)/gamma, layout private to the kernels). Every first
order derivative runs the HIP backward; jvp and derivatives of the backward
run ``_autograd`` through torch.func.
"""

from typing import Tuple

import torch
from torch import Tensor

from .. import _hip
from .._opsutil import (direct, jvp_of, per_pair_dot, pick, register_autocast, register_vmap,
                        vjp_of, without_jvp, zeros_if_none)
from . import _autograd

# ---------------------------------------------------- DP on given matrices


@torch.library.custom_op("twamd_udtw::dp", mutates_args=())
def dp(cost: Tensor, penalty: Tensor, gamma: float, bandwidth: float,
       backend: str) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    _hip.require(cost, backend, "uDTW")
    B, N, M = cost.shape
    c = cost.contiguous()
    pen = penalty.numel() > 0
    q = penalty.to(c.dtype).contiguous() if pen else None
    _hip.check_udtw_plane(N, M, gamma, c.dtype)
    R = c.new_empty(B, _hip.carry_cols(N, M, gamma, c.dtype))
    P = c.new_empty(B, N * M) if pen else c.new_empty(0)
    out_r, out_p = c.new_empty(B), c.new_empty(B)
    _hip.call("tw_udtw_cost_fwd", c.dtype, c, q, B, N, M, gamma, bandwidth, R, P, out_r, out_p)
    return out_r, out_p, R, P


@dp.register_fake
def _(cost, penalty, gamma, bandwidth, backend):
    B, N, M = cost.shape
    P = cost.new_empty(B, N * M) if penalty.numel() else cost.new_empty(0)
    R = cost.new_empty(B, _hip.carry_cols(N, M, gamma, cost.dtype))
    return cost.new_empty(B), cost.new_empty(B), R, P


@torch.library.custom_op("twamd_udtw::dp_backward", mutates_args=())
def dp_backward(cost: Tensor, penalty: Tensor, R: Tensor, P: Tensor, grad_r: Tensor,
                grad_p: Tensor, gamma: float, bandwidth: float,
                backend: str) -> Tuple[Tensor, Tensor]:
    _hip.require(cost, backend, "uDTW")
    B, N, M = cost.shape
    c = cost.contiguous()
    pen = penalty.numel() > 0
    q = penalty.to(c.dtype).contiguous() if pen else None
    d_cost = torch.empty_like(c)
    d_pen = torch.empty_like(c) if pen else c.new_empty(0)
    grads, gs = _hip.per_pair(*((grad_r.to(c.dtype), grad_p.to(c.dtype)) if pen
                                else (grad_r.to(c.dtype),)))
    nws = _hip.udtw_cost_workspace_elems(B, N, M, c.dtype, bandwidth)
    ws = c.new_empty(nws) if nws else c.new_empty(0)
    _hip.call("tw_udtw_cost_bwd", c.dtype, c, q, R, P, grads[0], grads[1] if pen else None,
              B, N, M, gamma, bandwidth, gs, d_cost, d_pen, *_ws_args(ws))
    return d_cost, d_pen


@dp_backward.register_fake
def _(cost, penalty, R, P, grad_r, grad_p, gamma, bandwidth, backend):
    return torch.empty_like(cost), (torch.empty_like(cost) if penalty.numel() else cost.new_empty(0))


register_vmap(dp, 2)
register_vmap(dp_backward, 6)
register_autocast(dp)
register_autocast(dp_backward)


# --------------------------------------------------------- from features


def _feat_ws(X, N, M, bandwidth):
    """The forward's plane [B, N*M]: the squared distances (D > 1) or, with a
    band narrower than the grid, the banded path's cost and penalty (D = 1
    too); empty when the forward needs none."""
    B, D = X.shape[0], X.shape[2]
    return (X.new_empty(B, N * M) if _hip.udtw_feat_plane(B, N, M, D, X.dtype, bandwidth)
            else X.new_empty(0))


def _feat_bwd_ws(X, N, M, bandwidth):
    """The backward's workspace: the squared-distance plane (D > 1) or the
    banded path's gradient planes, then the hand-off records of long
    sequences (empty when none is needed)."""
    n = _hip.udtw_workspace_elems(X.shape[0], N, M, X.shape[2], X.dtype, bandwidth)
    return X.new_empty(n) if n else X.new_empty(0)


def _ws_args(ws):
    return (ws, ws.numel() * ws.element_size()) if ws.numel() else (None, 0)


@torch.library.custom_op("twamd_udtw::fused", mutates_args=())
def fused(X: Tensor, Y: Tensor, vx: Tensor, vy: Tensor, gamma: float, beta: float, eps: float,
          bandwidth: float, backend: str,
          sigma: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """vx, vy: variances [B,N] / [B,M], or with ``sigma`` the standard deviations
    (any shape holding B*N / B*M values), squared inside the kernel. Returns
    (distance, penalty, R, P, S): S is the squared-distance plane the kernels
    built for D > 1 (empty for D == 1), which the backward reads instead of
    recomputing it."""
    _hip.require(X, backend, "uDTW")
    B, N, D = X.shape
    M = Y.shape[1]
    X, Y, vx, vy = _hip.dense(X.dtype, X, Y, vx, vy)
    pen = beta != 0.0
    _hip.check_udtw_plane(N, M, gamma, X.dtype)
    R = X.new_empty(B, _hip.carry_cols(N, M, gamma, X.dtype))
    P = X.new_empty(B, N * M) if pen else X.new_empty(0)
    out_r, out_p = X.new_empty(B), X.new_empty(B)
    S = _feat_ws(X, N, M, bandwidth)
    _hip.call("tw_udtw_feat_fwd", X.dtype, X, Y, vx, vy, B, N, M, D, gamma, beta, eps, bandwidth,
              int(sigma), R, P, out_r, out_p, *_ws_args(S))
    return out_r, out_p, R, P, S


@fused.register_fake
def _(X, Y, vx, vy, gamma, beta, eps, bandwidth, backend, sigma):
    B, N, M = X.shape[0], X.shape[1], Y.shape[1]
    P = X.new_empty(B, N * M) if beta != 0.0 else X.new_empty(0)
    S = _feat_ws(X, N, M, bandwidth)
    R = X.new_empty(B, _hip.carry_cols(N, M, gamma, X.dtype))
    return X.new_empty(B), X.new_empty(B), R, P, S


@torch.library.custom_op("twamd_udtw::fused_backward", mutates_args=())
def fused_backward(X: Tensor, Y: Tensor, vx: Tensor, vy: Tensor, R: Tensor, P: Tensor,
                   S: Tensor, grad_r: Tensor, grad_p: Tensor, gamma: float, beta: float, eps: float,
                   bandwidth: float, backend: str,
                   sigma: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    _hip.require(X, backend, "uDTW")
    B, N, D = X.shape
    M = Y.shape[1]
    X, Y, vx, vy = _hip.dense(X.dtype, X, Y, vx, vy)
    pen = beta != 0.0
    dX, dY = torch.empty_like(X), torch.empty_like(Y)
    dvx, dvy = torch.empty_like(vx), torch.empty_like(vy)
    ws = _feat_bwd_ws(X, N, M, bandwidth)
    S = S if (S.shape == (B, N * M) and S.dtype == X.dtype and S.is_contiguous()) else None
    grads, gs = _hip.per_pair(*(_hip.dense(X.dtype, grad_r, grad_p, contiguous=False) if pen
                                else _hip.dense(X.dtype, grad_r, contiguous=False)))
    _hip.call("tw_udtw_feat_bwd", X.dtype, X, Y, vx, vy, R, P if pen else None, grads[0],
              grads[1] if pen else None, B, N, M, D, gamma, beta, eps, bandwidth, int(sigma), gs,
              dX, dY, dvx, dvy, S, *_ws_args(ws))
    return dX, dY, dvx, dvy


@fused_backward.register_fake
def _(X, Y, vx, vy, R, P, S, grad_r, grad_p, gamma, beta, eps, bandwidth, backend, sigma):
    return torch.empty_like(X), torch.empty_like(Y), torch.empty_like(vx), torch.empty_like(vy)


register_vmap(fused, 4)
register_vmap(fused_backward, 9)
register_autocast(fused)
register_autocast(fused_backward)
_dp_direct = direct(dp)
_dp_backward_direct = direct(dp_backward)
_fused_direct = direct(fused)
_fused_backward_direct = direct(fused_backward)


# ------------------------------------------------------ autograd Functions


def _first_order(f, n):
    """(x_1..x_n, v_1..v_k) -> J_f(x)^T v, itself differentiable."""
    def g(*args):
        return vjp_of(f, args[:n], args[n:])
    return g


def _dense_pen(penalty, cost):
    return penalty if penalty.numel() else torch.zeros_like(cost)


class DP(torch.autograd.Function):
    """(cost, penalty) -> (distance, penalty_sum, R, P); R and P internal."""

    generate_vmap_rule = True

    @staticmethod
    def forward(cost, penalty, gamma, bandwidth, backend):
        return _dp_direct(cost, penalty, gamma, bandwidth, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        cost, penalty, gamma, bandwidth, backend = inputs
        ctx.mark_non_differentiable(output[2], output[3])
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(cost, penalty, output[2], output[3])
        ctx.save_for_forward(cost, penalty, output[2], output[3])
        ctx.args = (gamma, bandwidth, backend)

    @staticmethod
    def backward(ctx, g_r, g_p, _g_R, _g_P):
        cost, penalty, R, P = ctx.saved_tensors
        gamma, bandwidth, backend = ctx.args
        B = cost.shape[0]
        g_r = cost.new_zeros(B) if g_r is None else g_r
        g_p = cost.new_zeros(B) if g_p is None else g_p
        d_cost, d_pen = dp_backward_apply(cost, penalty, R, P, g_r, g_p, gamma, bandwidth, backend)
        return d_cost, d_pen, None, None, None

    @staticmethod
    def jvp(ctx, t_cost, t_pen, *_):
        # distance and penalty are one scalar per pair: their tangents are the
        # HIP backward's gradients (unit cotangent) dotted with the tangents
        cost, penalty, R, P = ctx.saved_tensors
        gamma, bandwidth, backend = ctx.args
        B = cost.shape[0]
        one, zero = cost.new_ones(B), cost.new_zeros(B)
        ts = (t_cost, t_pen if penalty.numel() else None)
        t_r = per_pair_dot(dp_backward_apply(cost, penalty, R, P, one, zero, gamma, bandwidth,
                                             backend), ts)
        t_p = None
        if penalty.numel():
            t_p = per_pair_dot(dp_backward_apply(cost, penalty, R, P, zero, one, gamma,
                                                 bandwidth, backend), ts)
        return (zero if t_r is None else t_r), (zero if t_p is None else t_p), None, None


class DPBackward(torch.autograd.Function):
    """First-order VJP of :class:`DP`; differentiable for higher orders."""

    generate_vmap_rule = True

    @staticmethod
    def forward(cost, penalty, R, P, g_r, g_p, gamma, bandwidth, backend):
        return _dp_backward_direct(cost, penalty, R, P, g_r, g_p, gamma, bandwidth, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        cost, penalty, R, P, g_r, g_p, gamma, bandwidth, backend = inputs
        ctx.save_for_backward(cost, penalty, g_r, g_p)
        ctx.save_for_forward(cost, penalty, g_r, g_p)
        ctx.args = (gamma, bandwidth)

    @staticmethod
    def _first(ctx):
        gamma, bandwidth = ctx.args
        return _first_order(lambda c, q: _autograd.udtw(c, q, gamma, bandwidth), 2)

    @staticmethod
    def backward(ctx, gg_cost, gg_pen):
        cost, penalty, g_r, g_p = ctx.saved_tensors
        pen = _dense_pen(penalty, cost)
        gg_pen = zeros_if_none(gg_pen, pen) if penalty.numel() else torch.zeros_like(cost)
        d = vjp_of(DPBackward._first(ctx), (cost, pen, g_r, g_p),
                   (zeros_if_none(gg_cost, cost), gg_pen))
        d_pen = d[1] if penalty.numel() else None
        return d[0], d_pen, None, None, d[2], d[3], None, None, None

    @staticmethod
    def jvp(ctx, t_cost, t_pen, _t_R, _t_P, t_gr, t_gp, *_):
        cost, penalty, g_r, g_p = ctx.saved_tensors
        pen = _dense_pen(penalty, cost)
        t_pen = zeros_if_none(t_pen, pen) if penalty.numel() else torch.zeros_like(cost)
        primals = (cost, pen, g_r, g_p)
        tangents = (zeros_if_none(t_cost, cost), t_pen, zeros_if_none(t_gr, g_r),
                    zeros_if_none(t_gp, g_p))
        out = jvp_of(DPBackward._first(ctx), primals, tangents)
        return out[0], (out[1] if penalty.numel() else penalty.new_empty(0))


def _variance(v, seq, sigma):
    """Variances [B, L] of the autograd-native path from a fused-op input."""
    v = v.reshape(seq.shape[0], seq.shape[1])
    return v * v if sigma else v


class Fused(torch.autograd.Function):
    """(X, Y, vx, vy) -> (distance, penalty_sum, R, P, S); R, P, S internal."""

    generate_vmap_rule = True

    @staticmethod
    def forward(X, Y, vx, vy, gamma, beta, eps, bandwidth, backend, sigma):
        return _fused_direct(X, Y, vx, vy, gamma, beta, eps, bandwidth, backend, sigma)

    @staticmethod
    def setup_context(ctx, inputs, output):
        X, Y, vx, vy, gamma, beta, eps, bandwidth, backend, sigma = inputs
        ctx.mark_non_differentiable(output[2], output[3], output[4])
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(X, Y, vx, vy, output[2], output[3], output[4])
        ctx.save_for_forward(X, Y, vx, vy, output[2], output[3], output[4])
        ctx.args = (gamma, beta, eps, bandwidth, backend, sigma)

    @staticmethod
    def backward(ctx, g_r, g_p, _g_R, _g_P, _g_S):
        X, Y, vx, vy, R, P, S = ctx.saved_tensors
        gamma, beta, eps, bandwidth, backend, sigma = ctx.args
        B = X.shape[0]
        g_r = X.new_zeros(B) if g_r is None else g_r
        g_p = X.new_zeros(B) if g_p is None else g_p
        grads = fused_backward_apply(X, Y, vx, vy, R, P, S, g_r, g_p, gamma, beta, eps,
                                     bandwidth, backend, sigma)
        return (*grads, None, None, None, None, None, None)

    @staticmethod
    def jvp(ctx, t_X, t_Y, t_vx, t_vy, *_):
        # one scalar per pair: gradients of the HIP backward (unit cotangent)
        # dotted with the tangents
        X, Y, vx, vy, R, P, S = ctx.saved_tensors
        gamma, beta, eps, bandwidth, backend, sigma = ctx.args
        B = X.shape[0]
        one, zero = X.new_ones(B), X.new_zeros(B)
        ts = (t_X, t_Y, t_vx, t_vy)
        args = (gamma, beta, eps, bandwidth, backend, sigma)
        t_r = per_pair_dot(fused_backward_apply(X, Y, vx, vy, R, P, S, one, zero, *args), ts)
        t_p = None
        if beta != 0.0:
            t_p = per_pair_dot(fused_backward_apply(X, Y, vx, vy, R, P, S, zero, one, *args), ts)
        return (zero if t_r is None else t_r), (zero if t_p is None else t_p), None, None, None


class FusedBackward(torch.autograd.Function):
    """First-order VJP of :class:`Fused`; differentiable for higher orders."""

    generate_vmap_rule = True

    @staticmethod
    def forward(X, Y, vx, vy, R, P, S, g_r, g_p, gamma, beta, eps, bandwidth, backend, sigma):
        return _fused_backward_direct(X, Y, vx, vy, R, P, S, g_r, g_p, gamma, beta, eps,
                                      bandwidth, backend, sigma)

    @staticmethod
    def setup_context(ctx, inputs, output):
        X, Y, vx, vy, R, P, S, g_r, g_p, gamma, beta, eps, bandwidth, backend, sigma = inputs
        ctx.save_for_backward(X, Y, vx, vy, g_r, g_p)
        ctx.save_for_forward(X, Y, vx, vy, g_r, g_p)
        ctx.args = (gamma, beta, eps, bandwidth, sigma)

    @staticmethod
    def _first(ctx):
        gamma, beta, eps, bandwidth, sigma = ctx.args
        return _first_order(
            lambda x, y, a, b: _autograd.udtw_features(x, y, _variance(a, x, sigma),
                                                       _variance(b, y, sigma), gamma, beta, eps,
                                                       bandwidth), 4)

    @staticmethod
    def backward(ctx, gg_X, gg_Y, gg_vx, gg_vy):
        X, Y, vx, vy, g_r, g_p = ctx.saved_tensors
        cot = tuple(zeros_if_none(g, p) for g, p in zip((gg_X, gg_Y, gg_vx, gg_vy), (X, Y, vx, vy)))
        d = vjp_of(FusedBackward._first(ctx), (X, Y, vx, vy, g_r, g_p), cot)
        return (d[0], d[1], d[2], d[3], None, None, None, d[4], d[5],
                None, None, None, None, None, None)

    @staticmethod
    def jvp(ctx, t_X, t_Y, t_vx, t_vy, _t_R, _t_P, _t_S, t_gr, t_gp, *_):
        primals = ctx.saved_tensors
        tangents = tuple(zeros_if_none(t, p) for t, p in
                         zip((t_X, t_Y, t_vx, t_vy, t_gr, t_gp), primals))
        return tuple(jvp_of(FusedBackward._first(ctx), primals, tangents))


dp_apply = pick(DP, without_jvp(DP), DP.forward)
dp_backward_apply = pick(DPBackward, without_jvp(DPBackward), DPBackward.forward)
fused_apply = pick(Fused, without_jvp(Fused), Fused.forward)
fused_backward_apply = pick(FusedBackward, without_jvp(FusedBackward), FusedBackward.forward)
