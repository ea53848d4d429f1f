"""The extended-precision uDTW restatement (oracle/udtw_ld.py), pinned, and the
float64 rounding floor it exposes at the long-sequence config (CPU only).

1. On small cases it equals the float64 oracle (itself pinned by the golden
   vectors) to ~1e-13, and its value equals the brute-force enumeration of
   every path.
2. At cfg3 (N = M = 1024, D = 16, gamma = 0.1), pair 0, the float64 oracle's
   gradients are ~1e-10 .. 1e-9 away from the extended-precision ones: the
   accumulated cost reaches ~2.7e4, so the backward weights
   exp((E_s - R_k) / gamma) inherit the float64 rounding of numbers of that
   size. Any float64 evaluation of this algorithm (the reference's included)
   carries that error; the GPU test test_cfg3_float64_against_extended_precision
   holds the HIP kernels to the same standard.
"""

import numpy as np
import pytest
import torch

from oracle import brute, udtw as OU, udtw_ld


def _f64(X, Y, vx, vy, gamma, beta):
    r, p, R, P = OU.features_forward(X[None], Y[None], vx[None], vy[None], gamma, beta, 1e-8)
    one = torch.ones(1, dtype=torch.float64)
    dX, dY, dvx, dvy = OU.features_backward(X[None], Y[None], vx[None], vy[None], R, P, one, one,
                                            gamma, beta, 1e-8)
    return [r[0], p[0], dX[0], dY[0], dvx[0], dvy[0]]


def _err(a, b):
    a = np.asarray(a.numpy() if isinstance(a, torch.Tensor) else a, np.longdouble).ravel()
    b = np.asarray(b, np.longdouble).ravel()
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.mark.parametrize("N, M, D, gamma, beta", [
    (1, 1, 2, 0.5, 1.0), (1, 6, 3, 0.3, 0.5), (7, 9, 3, 0.3, 0.7), (12, 10, 1, 1.0, 0.0),
    (20, 25, 4, 0.05, 2.0),
])
def test_extended_precision_equals_float64_oracle_on_small_cases(N, M, D, gamma, beta):
    g = torch.Generator().manual_seed(N * 100 + M)
    X = torch.randn(N, D, generator=g, dtype=torch.float64)
    Y = torch.randn(M, D, generator=g, dtype=torch.float64)
    vx = 0.5 + torch.rand(N, generator=g, dtype=torch.float64)
    vy = 0.5 + torch.rand(M, generator=g, dtype=torch.float64)
    want = _f64(X, Y, vx, vy, gamma, beta)
    got = udtw_ld.features_value_and_grads(X.numpy(), Y.numpy(), vx.numpy(), vy.numpy(), gamma,
                                           beta)
    for w, a in zip(want, got):
        assert _err(w, a) < 1e-12


def test_extended_precision_value_equals_path_enumeration():
    g = torch.Generator().manual_seed(3)
    X = torch.randn(3, 2, generator=g, dtype=torch.float64)
    Y = torch.randn(4, 2, generator=g, dtype=torch.float64)
    vx = 0.5 + torch.rand(3, generator=g, dtype=torch.float64)
    vy = 0.5 + torch.rand(4, generator=g, dtype=torch.float64)
    cost, pen, _, _ = OU.pairwise(X[None], Y[None], vx[None], vy[None], 0.6, 1e-8)
    want_r, want_p = brute.udtw_value(cost[0], pen[0], 0.4)
    r, p, *_ = udtw_ld.features_value_and_grads(X.numpy(), Y.numpy(), vx.numpy(), vy.numpy(),
                                                0.4, 0.6)
    assert abs(float(r) - want_r.item()) < 1e-13 * abs(want_r.item())
    assert abs(float(p) - want_p.item()) < 1e-13 * abs(want_p.item())


def test_float64_rounding_floor_at_cfg3():
    from bench import make_inputs
    X, Y, sx, sy = make_inputs("cfg3", dtype=torch.float64)
    X, Y, vx, vy = X[0], Y[0], sx[0, :, 0] ** 2, sy[0, :, 0] ** 2
    want = udtw_ld.features_value_and_grads(X.numpy(), Y.numpy(), vx.numpy(), vy.numpy(), 0.1,
                                            1.0)
    got = _f64(X, Y, vx, vy, 0.1, 1.0)
    errs = [_err(a, w) for a, w in zip(got, want)]
    print("\ncfg3 pair 0, float64 oracle vs extended precision:", ["%.2e" % e for e in errs])
    # values: cancellation-free sums, at float64 precision
    assert max(errs[:2]) < 1e-13
    # gradients: the float64 floor of the algorithm itself (measured 1.5e-10
    # .. 4.9e-10), clearly above float64 epsilon and clearly below 1e-8
    assert 1e-11 < max(errs[2:]) < 2e-9
