"""JEANIE, FVM and pairwise-cost custom operators over the HIP kernels, plus autograd Functions.

Operator contract of the reference (``jeanie/_ops.py:1-490``): custom ops
with fake implementations, vmap rules and float32 autocast; autograd
Functions with ``setup_context``, ``jvp`` and compiled twins. The accumulator
R is a differentiable output when requested (``natural_R``); first-order
reverse mode runs the HIP backward with dL/dR as an extra seed.

Ops (namespace ``twamd_*``):
* ``twamd_jeanie::dp`` / ``dp_backward`` -- cost path (reference
  ``torchwarp_jeanie::dp`` / ``dp_backward``, :110-139). The accumulator is
  kept in the cost's natural [B,K1,K2,T,U] layout, so it is both the tensor
  saved for the backward and the one returned to the caller: no layout
  permutation in either direction. T > U runs the transposed grid in place.
* ``twamd_jeanie::features`` / ``features_backward`` -- features path
  (``torchwarp_jeanie::features`` / ``features_backward``, :155-230): the
  pairwise cost is built by the HIP pair-cost kernel and saved; the backward
  maps d cost back to the query and support on the same kernels.
* ``twamd_fvm::fvm`` / ``fvm_backward`` -- ``fvm_from_cost``
  (``jeanie/fvm.py:15-38``): viewpoint softmin and soft-DTW in HIP.
* ``twamd_cost::pair`` / ``pair_backward`` -- (squared) Euclidean cost
  (``jeanie/distances.py:15-38``).
"""

from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _hip
from .._opsutil import (direct, jvp_of, per_pair_dot, pick, register_autocast, register_vmap,
                        vjp_of, without_jvp, zeros_if_none)
from . import _autograd

METRIC_CODES = {"sqeuclidean": _hip.METRIC_SQEUC, "euclidean": _hip.METRIC_EUC}


def _dp_dims(T, U):
    """(T_dp, U_dp, swap): the DP runs on the T <= U orientation."""
    return (U, T, 1) if T > U else (T, U, 0)


# ----------------------------------------------------------- pairwise cost

@torch.library.custom_op("twamd_cost::pair", mutates_args=())
def pair(A: Tensor, Bm: Tensor, metric: int, backend: str) -> Tensor:
    _hip.require(A, backend, "pairwise cost")
    P, R, D = A.shape
    C = Bm.shape[1]
    A, Bm = A.contiguous(), Bm.to(A.dtype).contiguous()
    out = A.new_empty(P, R, C)
    _hip.call("tw_pair_cost_fwd", A.dtype, A, Bm, P, R, C, D, metric, out)
    return out


@pair.register_fake
def _(A, Bm, metric, backend):
    return A.new_empty(A.shape[0], A.shape[1], Bm.shape[1])


@torch.library.custom_op("twamd_cost::pair_backward", mutates_args=())
def pair_backward(A: Tensor, Bm: Tensor, cost: Tensor, d_cost: Tensor, metric: int,
                  backend: str) -> Tuple[Tensor, Tensor]:
    _hip.require(A, backend, "pairwise cost")
    P, R, D = A.shape
    C = Bm.shape[1]
    A, Bm = A.contiguous(), Bm.to(A.dtype).contiguous()
    dA, dB = torch.empty_like(A), torch.empty_like(Bm)
    _hip.call("tw_pair_cost_bwd", A.dtype, A, Bm, cost.contiguous(),
              d_cost.to(A.dtype).contiguous(), P, R, C, D, metric, dA, dB)
    return dA, dB


@pair_backward.register_fake
def _(A, Bm, cost, d_cost, metric, backend):
    return torch.empty_like(A), torch.empty_like(Bm)


register_vmap(pair, 2)
register_vmap(pair_backward, 4)
register_autocast(pair)
register_autocast(pair_backward)


class Pair(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(A, Bm, metric, backend):
        return _pair_direct(A, Bm, metric, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        A, Bm, metric, backend = inputs
        ctx.save_for_backward(A, Bm, output)
        ctx.save_for_forward(A, Bm)
        ctx.args = (metric, backend)

    @staticmethod
    def backward(ctx, g):
        A, Bm, cost = ctx.saved_tensors
        metric, backend = ctx.args
        dA, dB = pair_backward_apply(A, Bm, cost, g, metric, backend)
        return dA, dB, None, None

    @staticmethod
    def jvp(ctx, tA, tB, *_):
        A, Bm = ctx.saved_tensors
        metric, _ = ctx.args
        return jvp_of(lambda a, b: _autograd.pair_cost(a, b, metric), (A, Bm),
                      (zeros_if_none(tA, A), zeros_if_none(tB, Bm)))


class PairBackward(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(A, Bm, cost, g, metric, backend):
        return _pair_backward_direct(A, Bm, cost, g, metric, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        A, Bm, cost, g, metric, backend = inputs
        ctx.save_for_backward(A, Bm, g)
        ctx.save_for_forward(A, Bm, g)
        ctx.metric = metric

    @staticmethod
    def _first(metric):
        return lambda a, b, g: vjp_of(lambda x, y: _autograd.pair_cost(x, y, metric), (a, b), (g,))

    @staticmethod
    def backward(ctx, gg_A, gg_B):
        A, Bm, g = ctx.saved_tensors
        d = vjp_of(PairBackward._first(ctx.metric), (A, Bm, g),
                   (zeros_if_none(gg_A, A), zeros_if_none(gg_B, Bm)))
        return d[0], d[1], None, d[2], None, None

    @staticmethod
    def jvp(ctx, tA, tB, _tc, tg, *_):
        A, Bm, g = ctx.saved_tensors
        tangents = tuple(zeros_if_none(t, p) for t, p in zip((tA, tB, tg), (A, Bm, g)))
        return tuple(jvp_of(PairBackward._first(ctx.metric), (A, Bm, g), tangents))


pair_apply = pick(Pair, without_jvp(Pair), Pair.forward)
pair_backward_apply = pick(PairBackward, without_jvp(PairBackward), PairBackward.forward)


# -------------------------------------------------------------- RBF cost

@torch.library.custom_op("twamd_cost::rbf", mutates_args=())
def rbf(A: Tensor, Bm: Tensor, sigma: float, backend: str) -> Tensor:
    _hip.require(A, backend, "rbf cost")
    P, R, D = A.shape
    C = Bm.shape[1]
    A, Bm = A.contiguous(), Bm.to(A.dtype).contiguous()
    out = A.new_empty(P, R, C)
    _hip.call("tw_rbf_cost_fwd", A.dtype, A, Bm, P, R, C, D, sigma, out)
    return out


@rbf.register_fake
def _(A, Bm, sigma, backend):
    return A.new_empty(A.shape[0], A.shape[1], Bm.shape[1])


@torch.library.custom_op("twamd_cost::rbf_backward", mutates_args=())
def rbf_backward(A: Tensor, Bm: Tensor, d_cost: Tensor, sigma: float,
                 backend: str) -> Tuple[Tensor, Tensor]:
    _hip.require(A, backend, "rbf cost")
    P, R, D = A.shape
    C = Bm.shape[1]
    A, Bm = A.contiguous(), Bm.to(A.dtype).contiguous()
    dA, dB = torch.empty_like(A), torch.empty_like(Bm)
    _hip.call("tw_rbf_cost_bwd", A.dtype, A, Bm, d_cost.to(A.dtype).contiguous(), P, R, C, D,
              sigma, dA, dB)
    return dA, dB


@rbf_backward.register_fake
def _(A, Bm, d_cost, sigma, backend):
    return torch.empty_like(A), torch.empty_like(Bm)


register_vmap(rbf, 2)
register_vmap(rbf_backward, 3)
register_autocast(rbf)
register_autocast(rbf_backward)


class Rbf(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(A, Bm, sigma, backend):
        return _rbf_direct(A, Bm, sigma, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        A, Bm, sigma, backend = inputs
        ctx.save_for_backward(A, Bm)
        ctx.save_for_forward(A, Bm)
        ctx.args = (sigma, backend)

    @staticmethod
    def backward(ctx, g):
        A, Bm = ctx.saved_tensors
        sigma, backend = ctx.args
        dA, dB = rbf_backward_apply(A, Bm, g, sigma, backend)
        return dA, dB, None, None

    @staticmethod
    def jvp(ctx, tA, tB, *_):
        A, Bm = ctx.saved_tensors
        sigma, _ = ctx.args
        return jvp_of(lambda a, b: _autograd.rbf_cost(a, b, sigma), (A, Bm),
                      (zeros_if_none(tA, A), zeros_if_none(tB, Bm)))


class RbfBackward(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(A, Bm, g, sigma, backend):
        return _rbf_backward_direct(A, Bm, g, sigma, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        A, Bm, g, sigma, backend = inputs
        ctx.save_for_backward(A, Bm, g)
        ctx.save_for_forward(A, Bm, g)
        ctx.sigma = sigma

    @staticmethod
    def _first(sigma):
        return lambda a, b, g: vjp_of(lambda x, y: _autograd.rbf_cost(x, y, sigma), (a, b), (g,))

    @staticmethod
    def backward(ctx, gg_A, gg_B):
        A, Bm, g = ctx.saved_tensors
        d = vjp_of(RbfBackward._first(ctx.sigma), (A, Bm, g),
                   (zeros_if_none(gg_A, A), zeros_if_none(gg_B, Bm)))
        return d[0], d[1], d[2], None, None

    @staticmethod
    def jvp(ctx, tA, tB, tg, *_):
        A, Bm, g = ctx.saved_tensors
        tangents = tuple(zeros_if_none(t, p) for t, p in zip((tA, tB, tg), (A, Bm, g)))
        return tuple(jvp_of(RbfBackward._first(ctx.sigma), (A, Bm, g), tangents))


rbf_apply = pick(Rbf, without_jvp(Rbf), Rbf.forward)
rbf_backward_apply = pick(RbfBackward, without_jvp(RbfBackward), RbfBackward.forward)


# ----------------------------------------------------------- JEANIE, cost

@torch.library.custom_op("twamd_jeanie::dp", mutates_args=())
def dp(cost: Tensor, s1: int, s2: int, gamma: float, backend: str) -> Tuple[Tensor, Tensor]:
    _hip.require(cost, backend, "JEANIE")
    c = cost.contiguous()
    B, K1, K2, T, U = c.shape
    Td, Ud, swap = _dp_dims(T, U)
    R, out = torch.empty_like(c), c.new_empty(B)
    _hip.call("tw_jeanie_cost_fwd", c.dtype, c, B, K1, K2, Td, Ud, swap, s1, s2, gamma, R, out)
    return out, R


@dp.register_fake
def _(cost, s1, s2, gamma, backend):
    return cost.new_empty(cost.shape[0]), torch.empty_like(cost)


@torch.library.custom_op("twamd_jeanie::dp_backward", mutates_args=())
def dp_backward(cost: Tensor, R: Tensor, grad_out: Tensor, grad_R: Optional[Tensor], s1: int,
                s2: int, gamma: float, backend: str) -> Tensor:
    _hip.require(cost, backend, "JEANIE")
    c = cost.contiguous()
    B, K1, K2, T, U = c.shape
    Td, Ud, swap = _dp_dims(T, U)
    gR = None if grad_R is None else grad_R.to(c.dtype).contiguous()
    d = torch.empty_like(c)
    _hip.call("tw_jeanie_cost_bwd", c.dtype, c, R.contiguous(), grad_out.to(c.dtype).contiguous(),
              gR, B, K1, K2, Td, Ud, swap, s1, s2, gamma, d)
    return d


@dp_backward.register_fake
def _(cost, R, grad_out, grad_R, s1, s2, gamma, backend):
    return torch.empty_like(cost)


register_vmap(dp, 1)
register_vmap(dp_backward, 4)
register_autocast(dp)
register_autocast(dp_backward)


def _r_grad(g, natural_R):
    return g if (natural_R and g is not None and g.numel()) else None


class DP(torch.autograd.Function):
    """cost -> (out, R); R is the accumulator, differentiable when ``natural_R``."""

    generate_vmap_rule = True

    @staticmethod
    def forward(cost, s1, s2, gamma, backend, natural_R):
        return _dp_direct(cost, s1, s2, gamma, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        cost, s1, s2, gamma, backend, natural_R = inputs
        if not natural_R:
            ctx.mark_non_differentiable(output[1])
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(cost, output[1])
        ctx.save_for_forward(cost, output[1])
        ctx.args = (s1, s2, gamma, backend, natural_R)

    @staticmethod
    def backward(ctx, g_out, g_R):
        cost, R = ctx.saved_tensors
        s1, s2, gamma, backend, natural_R = ctx.args
        g_out = cost.new_zeros(cost.shape[0]) if g_out is None else g_out
        d = dp_backward_apply(cost, R, g_out, _r_grad(g_R, natural_R), s1, s2, gamma, backend)
        return d, None, None, None, None, None

    @staticmethod
    def jvp(ctx, t_cost, *_):
        cost, R = ctx.saved_tensors
        s1, s2, gamma, backend, natural_R = ctx.args
        if natural_R:
            # the accumulator is an output too: forward mode through the
            # autograd-native recursion
            return jvp_of(lambda c: _autograd.jeanie(c, s1, s2, gamma), (cost,),
                          (zeros_if_none(t_cost, cost),))
        # one scalar per pair: the HIP backward's gradient (unit cotangent)
        # dotted with the tangent
        one = cost.new_ones(cost.shape[0])
        t_out = per_pair_dot((dp_backward_apply(cost, R, one, None, s1, s2, gamma, backend),),
                             (t_cost,))
        return (torch.zeros_like(one) if t_out is None else t_out), None


def _first_order_dp(s1, s2, gamma, with_R):
    def f(c):
        return _autograd.jeanie(c, s1, s2, gamma)
    if with_R:
        return lambda c, go, gR: vjp_of(f, (c,), (go, gR))
    return lambda c, go: vjp_of(lambda c: (f(c)[0],), (c,), (go,))


class DPBackward(torch.autograd.Function):
    """First-order VJP of :class:`DP`; differentiable for higher orders."""

    generate_vmap_rule = True

    @staticmethod
    def forward(cost, R, g_out, g_R, s1, s2, gamma, backend):
        return _dp_backward_direct(cost, R, g_out, g_R, s1, s2, gamma, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        cost, R, g_out, g_R, s1, s2, gamma, backend = inputs
        saved = (cost, g_out) if g_R is None else (cost, g_out, g_R)
        ctx.save_for_backward(*saved)
        ctx.save_for_forward(*saved)
        ctx.args = (s1, s2, gamma)
        ctx.with_R = g_R is not None

    @staticmethod
    def backward(ctx, gg):
        saved = ctx.saved_tensors
        d = vjp_of(_first_order_dp(*ctx.args, ctx.with_R), saved, (zeros_if_none(gg, saved[0]),))
        return d[0], None, d[1], (d[2] if ctx.with_R else None), None, None, None, None

    @staticmethod
    def jvp(ctx, t_cost, _t_R, t_go, t_gR, *_):
        saved = ctx.saved_tensors
        tangents = (t_cost, t_go, t_gR)[:len(saved)]
        tangents = tuple(zeros_if_none(t, p) for t, p in zip(tangents, saved))
        return jvp_of(_first_order_dp(*ctx.args, ctx.with_R), saved, tangents)[0]


dp_apply = pick(DP, without_jvp(DP), DP.forward)
dp_backward_apply = pick(DPBackward, without_jvp(DPBackward), DPBackward.forward)


# ------------------------------------------------------- JEANIE, features

@torch.library.custom_op("twamd_jeanie::features", mutates_args=())
def features(query: Tensor, support: Tensor, s1: int, s2: int, gamma: float, metric: int,
             backend: str) -> Tuple[Tensor, Tensor, Tensor]:
    _hip.require(query, backend, "JEANIE")
    q = query.contiguous()
    s = support.to(q.dtype).contiguous()
    B, K1, K2, T, D = q.shape
    U = s.shape[1]
    cost = q.new_empty(B, K1, K2, T, U)
    R, out = torch.empty_like(cost), q.new_empty(B)
    _hip.call("tw_jeanie_feat_fwd", q.dtype, q, s, B, K1, K2, T, U, D, s1, s2, gamma, metric,
              cost, R, out)
    return out, R, cost


@features.register_fake
def _(query, support, s1, s2, gamma, metric, backend):
    B, K1, K2, T, D = query.shape
    U = support.shape[1]
    return (query.new_empty(B), query.new_empty(B, K1, K2, T, U),
            query.new_empty(B, K1, K2, T, U))


@torch.library.custom_op("twamd_jeanie::features_backward", mutates_args=())
def features_backward(query: Tensor, support: Tensor, cost: Tensor, R: Tensor, grad_out: Tensor,
                      grad_R: Optional[Tensor], s1: int, s2: int, gamma: float, metric: int,
                      backend: str) -> Tuple[Tensor, Tensor]:
    _hip.require(query, backend, "JEANIE")
    q = query.contiguous()
    s = support.to(q.dtype).contiguous()
    B, K1, K2, T, D = q.shape
    U = s.shape[1]
    gR = None if grad_R is None else grad_R.to(q.dtype).contiguous()
    dq, ds = torch.empty_like(q), torch.empty_like(s)
    ws = torch.empty_like(cost)
    _hip.call("tw_jeanie_feat_bwd", q.dtype, q, s, cost.contiguous(), R.contiguous(),
              grad_out.to(q.dtype).contiguous(), gR, B, K1, K2, T, U, D, s1, s2, gamma, metric,
              dq, ds, ws)
    return dq, ds


@features_backward.register_fake
def _(query, support, cost, R, grad_out, grad_R, s1, s2, gamma, metric, backend):
    return torch.empty_like(query), torch.empty_like(support)


register_vmap(features, 2)
register_vmap(features_backward, 6)
register_autocast(features)
register_autocast(features_backward)


def _first_order_features(s1, s2, gamma, metric, with_R):
    def f(q, s):
        return _autograd.jeanie_features(q, s, s1, s2, gamma, metric)
    if with_R:
        return lambda q, s, go, gR: tuple(vjp_of(f, (q, s), (go, gR)))
    return lambda q, s, go: tuple(vjp_of(lambda q, s: (f(q, s)[0],), (q, s), (go,)))


class Features(torch.autograd.Function):
    """(query, support) -> (out, R, cost); R differentiable when ``natural_R``."""

    generate_vmap_rule = True

    @staticmethod
    def forward(query, support, s1, s2, gamma, metric, backend, natural_R):
        return _features_direct(query, support, s1, s2, gamma, metric, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        query, support, s1, s2, gamma, metric, backend, natural_R = inputs
        out, R, cost = output
        if natural_R:
            ctx.mark_non_differentiable(cost)
        else:
            ctx.mark_non_differentiable(R, cost)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(query, support, cost, R)
        ctx.save_for_forward(query, support, cost, R)
        ctx.args = (s1, s2, gamma, metric, backend, natural_R)

    @staticmethod
    def backward(ctx, g_out, g_R, _g_cost):
        query, support, cost, R = ctx.saved_tensors
        s1, s2, gamma, metric, backend, natural_R = ctx.args
        g_out = query.new_zeros(query.shape[0]) if g_out is None else g_out
        dq, ds = features_backward_apply(query, support, cost, R, g_out, _r_grad(g_R, natural_R),
                                         s1, s2, gamma, metric, backend)
        return dq, ds, None, None, None, None, None, None

    @staticmethod
    def jvp(ctx, t_q, t_s, *_):
        query, support, cost, R = ctx.saved_tensors
        s1, s2, gamma, metric, backend, natural_R = ctx.args
        if natural_R:
            t_out, t_R = jvp_of(
                lambda q, s: _autograd.jeanie_features(q, s, s1, s2, gamma, metric),
                (query, support), (zeros_if_none(t_q, query), zeros_if_none(t_s, support)))
            return t_out, t_R, None
        one = query.new_ones(query.shape[0])
        grads = features_backward_apply(query, support, cost, R, one, None, s1, s2, gamma,
                                        metric, backend)
        t_out = per_pair_dot(grads, (t_q, t_s))
        return (torch.zeros_like(one) if t_out is None else t_out), None, None


class FeaturesBackward(torch.autograd.Function):
    """First-order VJP of :class:`Features`; differentiable for higher orders."""

    generate_vmap_rule = True

    @staticmethod
    def forward(query, support, cost, R, g_out, g_R, s1, s2, gamma, metric, backend):
        return _features_backward_direct(query, support, cost, R, g_out, g_R, s1, s2, gamma, metric,
                                 backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        query, support, cost, R, g_out, g_R, s1, s2, gamma, metric, backend = inputs
        saved = (query, support, g_out) if g_R is None else (query, support, g_out, g_R)
        ctx.save_for_backward(*saved)
        ctx.save_for_forward(*saved)
        ctx.args = (s1, s2, gamma, metric)
        ctx.with_R = g_R is not None

    @staticmethod
    def backward(ctx, gg_q, gg_s):
        saved = ctx.saved_tensors
        d = vjp_of(_first_order_features(*ctx.args, ctx.with_R), saved,
                   (zeros_if_none(gg_q, saved[0]), zeros_if_none(gg_s, saved[1])))
        d_gR = d[3] if ctx.with_R else None
        return d[0], d[1], None, None, d[2], d_gR, None, None, None, None, None

    @staticmethod
    def jvp(ctx, t_q, t_s, _t_c, _t_R, t_go, t_gR, *_):
        saved = ctx.saved_tensors
        tangents = (t_q, t_s, t_go, t_gR)[:len(saved)]
        tangents = tuple(zeros_if_none(t, p) for t, p in zip(tangents, saved))
        return jvp_of(_first_order_features(*ctx.args, ctx.with_R), saved, tangents)


features_apply = pick(Features, without_jvp(Features), Features.forward)
features_backward_apply = pick(FeaturesBackward, without_jvp(FeaturesBackward),
                               FeaturesBackward.forward)


# ------------------------------------------------------------------- FVM

@torch.library.custom_op("twamd_fvm::fvm", mutates_args=())
def fvm(cost: Tensor, gamma: float, backend: str) -> Tuple[Tensor, Tensor, Tensor]:
    _hip.require(cost, backend, "FVM")
    c = cost.contiguous()
    B, K, T, U = c.shape
    temporal, R = c.new_empty(B, T * U), c.new_empty(B, T * U)
    out, scratch = c.new_empty(B), c.new_empty(B)
    _hip.call("tw_fvm_cost_fwd", c.dtype, c, B, K, T, U, gamma, temporal, R, out, scratch)
    return out, temporal, R


@fvm.register_fake
def _(cost, gamma, backend):
    B, K, T, U = cost.shape
    return cost.new_empty(B), cost.new_empty(B, T * U), cost.new_empty(B, T * U)


@torch.library.custom_op("twamd_fvm::fvm_backward", mutates_args=())
def fvm_backward(cost: Tensor, temporal: Tensor, R: Tensor, grad_out: Tensor, gamma: float,
                 backend: str) -> Tensor:
    _hip.require(cost, backend, "FVM")
    c = cost.contiguous()
    B, K, T, U = c.shape
    es = c.element_size()
    nws = -(-_hip.library().tw_fvm_workspace_bytes(B, K, T, U, es) // es)
    d, ws = torch.empty_like(c), c.new_empty(nws)
    _hip.call("tw_fvm_cost_bwd", c.dtype, c, temporal, R, grad_out.to(c.dtype).contiguous(), B, K,
              T, U, gamma, d, ws, nws * es)
    return d


@fvm_backward.register_fake
def _(cost, temporal, R, grad_out, gamma, backend):
    return torch.empty_like(cost)


register_vmap(fvm, 1)
register_vmap(fvm_backward, 4)
register_autocast(fvm)
register_autocast(fvm_backward)
_pair_direct = direct(pair)
_pair_backward_direct = direct(pair_backward)
_rbf_direct = direct(rbf)
_rbf_backward_direct = direct(rbf_backward)
_dp_direct = direct(dp)
_dp_backward_direct = direct(dp_backward)
_features_direct = direct(features)
_features_backward_direct = direct(features_backward)
_fvm_direct = direct(fvm)
_fvm_backward_direct = direct(fvm_backward)


class FVM(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(cost, gamma, backend):
        return _fvm_direct(cost, gamma, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        cost, gamma, backend = inputs
        ctx.mark_non_differentiable(output[1], output[2])
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(cost, output[1], output[2])
        ctx.save_for_forward(cost, output[1], output[2])
        ctx.args = (gamma, backend)

    @staticmethod
    def backward(ctx, g_out, _gt, _gR):
        cost, temporal, R = ctx.saved_tensors
        gamma, backend = ctx.args
        if g_out is None:
            return None, None, None
        return fvm_backward_apply(cost, temporal, R, g_out, gamma, backend), None, None

    @staticmethod
    def jvp(ctx, t_cost, *_):
        # one scalar per pair: the HIP backward's gradient dotted with the tangent
        cost, temporal, R = ctx.saved_tensors
        gamma, backend = ctx.args
        one = cost.new_ones(cost.shape[0])
        t_out = per_pair_dot((fvm_backward_apply(cost, temporal, R, one, gamma, backend),),
                             (t_cost,))
        return (torch.zeros_like(one) if t_out is None else t_out), None, None


class FVMBackward(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(cost, temporal, R, g_out, gamma, backend):
        return _fvm_backward_direct(cost, temporal, R, g_out, gamma, backend)

    @staticmethod
    def setup_context(ctx, inputs, output):
        cost, temporal, R, g_out, gamma, backend = inputs
        ctx.save_for_backward(cost, g_out)
        ctx.save_for_forward(cost, g_out)
        ctx.gamma = gamma

    @staticmethod
    def _first(gamma):
        return lambda c, go: vjp_of(lambda x: (_autograd.fvm(x, gamma),), (c,), (go,))[0]

    @staticmethod
    def backward(ctx, gg):
        cost, g_out = ctx.saved_tensors
        d = vjp_of(FVMBackward._first(ctx.gamma), (cost, g_out), (zeros_if_none(gg, cost),))
        return d[0], None, None, d[1], None, None

    @staticmethod
    def jvp(ctx, t_cost, _tt, _tR, t_go, *_):
        cost, g_out = ctx.saved_tensors
        return jvp_of(FVMBackward._first(ctx.gamma), (cost, g_out),
                      (zeros_if_none(t_cost, cost), zeros_if_none(t_go, g_out)))


fvm_apply = pick(FVM, without_jvp(FVM), FVM.forward)
fvm_backward_apply = pick(FVMBackward, without_jvp(FVMBackward), FVMBackward.forward)
