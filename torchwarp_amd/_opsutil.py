"""Shared plumbing of the custom operators: vmap rules, autocast, derivative helpers.

Same operator contract as the reference (``udtw/_ops.py:60-95``,
``jeanie/_ops.py:67-105``): each op folds a vmapped dimension into its batch
dimension, runs in float32 under autocast, and the ``autograd.Function``
wrappers route first-order reverse mode to the HIP backward op while forward
mode and derivatives of a backward go through ``torch.func`` on the
autograd-native restatement.
"""

import torch
from torch import Tensor
from torch.autograd import forward_ad as _fwad


def register_vmap(op, n_tensors):
    """vmap rule: fold the vmapped dimension into the leading batch dimension."""
    def rule(info, in_dims, *args):
        V = info.batch_size
        folded = []
        for k, (a, d) in enumerate(zip(args, in_dims)):
            if k < n_tensors and isinstance(a, Tensor):
                a = a.unsqueeze(0).expand(V, *a.shape) if d is None else a.movedim(d, 0)
                a = a.reshape(V * a.shape[1], *a.shape[2:]).contiguous()
            folded.append(a)
        outs = op(*folded)
        single = not isinstance(outs, tuple)
        outs = (outs,) if single else outs
        outs = tuple(o.reshape(V, o.shape[0] // V, *o.shape[1:]) if o.numel() else o.new_empty(V, 0)
                     for o in outs)
        if single:
            return outs[0], 0
        return outs, tuple(0 for _ in outs)
    op.register_vmap(rule)


def register_autocast(op):
    for device in ("cuda", "cpu"):
        torch.library.register_autocast(op, device, torch.float32)


def zeros_if_none(g, like):
    return torch.zeros_like(like) if g is None else g


def jvp_of(f, primals, tangents):
    """J t of f at primals (inputs made dense: jacrev hands over expanded tensors)."""
    primals = tuple(p.contiguous() for p in primals)
    tangents = tuple(t.contiguous() for t in tangents)
    return torch.func.jvp(f, primals, tangents)[1]


def vjp_of(f, primals, cotangents):
    """J^T v of f at primals, itself differentiable. For an f with one tensor
    output, the one cotangent is passed as that tensor (torch.func matches
    the cotangents' structure to the outputs')."""
    out, pullback = torch.func.vjp(f, *primals)
    cot = tuple(cotangents)
    if isinstance(out, Tensor) and len(cot) == 1:
        return pullback(cot[0])
    return pullback(cot)


def per_pair_dot(grads, tangents):
    """sum_b-wise <grad, tangent>: for outputs with one scalar per pair b,
    whose gradient with respect to pair b's inputs is the VJP with a unit
    cotangent, this is the JVP (forward-mode derivative) of that output.
    Tangents given as None are skipped; None if every one is."""
    out = None
    for g, t in zip(grads, tangents):
        if g is None or t is None:
            continue
        v = g * t
        v = v.reshape(v.shape[0], -1).sum(1) if v.numel() else v.new_zeros(v.shape[0])
        out = v if out is None else out + v
    return out


def without_jvp(cls):
    """Twin of an autograd.Function without ``jvp`` (dynamo cannot trace one that has it)."""
    ns = {k: v for k, v in vars(cls).items() if k not in ("jvp", "__dict__", "__weakref__")}
    return type(cls.__name__ + "Compiled", (torch.autograd.Function,), ns)


_PLAIN = (Tensor, torch.nn.Parameter)


def plain_eager(args):
    """True for a call that no tracing, transform, mode or autocast can observe:
    not compiling, no functorch transform, no dispatch / torch-function mode,
    autocast off, and only plain tensors among the arguments."""
    if torch.compiler.is_compiling() or torch._C._are_functorch_transforms_active():
        return False
    if torch._C._len_torch_dispatch_stack() or torch._C._is_torch_function_mode_enabled():
        return False
    if torch.is_autocast_enabled("cuda") or torch.is_autocast_enabled("cpu"):
        return False
    return all(type(a) in _PLAIN for a in args if isinstance(a, Tensor))


def direct(op):
    """Call a custom op; in plain eager mode call its implementation directly.

    The op (fake kernel, vmap rule, autocast) serves every traced or
    transformed call; a plain eager call gets the same implementation without
    the dispatcher round trip.
    """
    impl = op._init_fn

    def call(*args):
        if plain_eager(args):
            return impl(*args)
        return op(*args)
    return call


def _records_nothing(args):
    """True when ``Function.apply`` would record no graph: grad mode off, no
    forward-mode dual level entered, and a plain eager call (as for
    :func:`plain_eager`). The backward of a first-order ``backward()`` runs
    this way, so its VJP Function then reduces to its forward."""
    if torch.is_grad_enabled() or _fwad._current_level >= 0:
        return False
    return plain_eager(args)


def pick(cls, compiled, forward=None):
    """``cls.apply``, with the compiled twin while torch.compile traces.

    With all arguments given positionally and no functorch transform active,
    ``Function.apply`` only adds a per-call ``inspect.signature`` binding of
    default arguments before the C++ apply; the plain path calls the C++
    apply directly (dead functorch wrappers are still unwrapped). When
    ``forward`` (the Function's forward) is given and the call records
    nothing (:func:`_records_nothing`), it is called directly.
    """
    base_apply = super(torch.autograd.Function, cls).apply
    unwrap = torch._functorch.utils.unwrap_if_dead

    def apply(*args):
        if torch.compiler.is_compiling():
            return compiled.apply(*args)
        if torch._C._are_functorch_transforms_active():
            return cls.apply(*args)
        if forward is not None and _records_nothing(args):
            return forward(*args)
        return base_apply(*[unwrap(a) if isinstance(a, Tensor) else a for a in args])
    return apply
