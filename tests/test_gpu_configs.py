"""HIP path vs the CPU oracle at the BASELINE config shapes (same seeded inputs).

float64: values and gradients within 1e-10 relative to the largest entry.
float32: max-normalised error against the float64 oracle (the reference's own
accuracy metric, tests/test_udtw.py:135), gated at the tolerances below and
printed for the record.
"""

import pytest
import torch

from bench import make_inputs
from oracle import jeanie as OJ, udtw as OU
import torchwarp_amd as tw
import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"
F64_TOL = 1e-10
F32_VALUE_TOL = 1e-5   # distances, relative to the largest distance
# Gradients, relative to the largest gradient entry. float32 stores R with an
# absolute rounding of ulp(|R|); at cfg2 |R| reaches ~70 (scaled), so every
# backward weight carries ~4e-6 relative error and ~280 chained diagonals give
# ~1e-4 -- the same floor as the reference's own float32 kernel.
F32_GRAD_TOL = 2e-4


def maxnorm_err(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


def _udtw_oracle(X, Y, sx, sy, gamma, beta):
    """fp64 oracle: distance, penalty and the gradients of mean(d + p)."""
    X, Y, sx, sy = (t.double() for t in (X, Y, sx, sy))
    vx, vy = sx.squeeze(-1) ** 2, sy.squeeze(-1) ** 2
    r, p, R, P = OU.features_forward(X, Y, vx, vy, gamma, beta, 1e-8)
    B = X.shape[0]
    g = torch.full((B,), 1.0 / B, dtype=torch.float64)
    dX, dY, dvx, dvy = OU.features_backward(X, Y, vx, vy, R, P, g, g if beta else 0 * g, gamma,
                                            beta, 1e-8)
    return [r, p, dX, dY, (2 * sx.squeeze(-1) * dvx).unsqueeze(-1),
            (2 * sy.squeeze(-1) * dvy).unsqueeze(-1)]


def _udtw_gpu(X, Y, sx, sy, gamma, beta, dtype):
    xs = [t.to(DEV, dtype).requires_grad_(True) for t in (X, Y, sx, sy)]
    d, p = tw.UDTW(gamma=gamma, beta=beta)(*xs)
    (d + p).mean().backward()
    return [d, p] + [t.grad for t in xs]


def _check(got, want, dtype, label):
    errs = [maxnorm_err(a, b) for a, b in zip(got, want)]
    print("\n{} {}: max-normalised errors {}".format(label, dtype, ["%.2e" % e for e in errs]))
    for k, e in enumerate(errs):
        if dtype == torch.float64:
            assert e < F64_TOL, (label, k, e)
        else:
            assert e < (F32_VALUE_TOL if k < 2 else F32_GRAD_TOL), (label, k, e)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_cfg2_udtw(dtype):
    X, Y, sx, sy = make_inputs("cfg2", dtype=torch.float64)
    _check(_udtw_gpu(X, Y, sx, sy, 1.0, 1.0, dtype), _udtw_oracle(X, Y, sx, sy, 1.0, 1.0),
           dtype, "cfg2")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_cfg1_soft_dtw(dtype):
    X, Y = make_inputs("cfg1", dtype=torch.float64)
    x = X.to(DEV, dtype).requires_grad_(True)
    d = tw.SoftDTW(gamma=1.0)(x, Y.to(DEV, dtype))
    d.mean().backward()
    ones = torch.ones(X.shape[0], X.shape[1], 1, dtype=torch.float64)
    want = _udtw_oracle(X, Y, ones, torch.ones(Y.shape[0], Y.shape[1], 1, dtype=torch.float64),
                        1.0, 0.0)
    _check([d, x.grad], [want[0], want[2]], dtype, "cfg1")


# cfg3: the launch is the full batch (64 pairs); the float64 oracle checks
# the first CFG3_CHECKED of them (each takes ~1.5 s on one CPU thread), with
# the gradient of the full batch's mean (1/64 per pair).
CFG3_CHECKED = 8


def _cfg3(beta):
    X, Y, sx, sy = make_inputs("cfg3", dtype=torch.float64)
    if beta == 0.0:   # soft-DTW: sigma = 1
        sx, sy = torch.ones_like(sx), torch.ones_like(sy)
    return X, Y, sx, sy


def _cfg3_gpu(X, Y, sx, sy, beta, dtype):
    if beta == 0.0:
        x, y = (t.to(DEV, dtype).requires_grad_(True) for t in (X, Y))
        d = tw.SoftDTW(gamma=0.1)(x, y)
        d.mean().backward()
        return [d, torch.zeros_like(d), x.grad, y.grad]
    got = _udtw_gpu(X, Y, sx, sy, 0.1, beta, dtype)
    return got[:4]


def _cfg3_oracle(X, Y, sx, sy, beta, k):
    X, Y, sx, sy = (t[:k] for t in (X, Y, sx, sy))
    vx, vy = sx.squeeze(-1) ** 2, sy.squeeze(-1) ** 2
    r, p, R, P = OU.features_forward(X, Y, vx, vy, 0.1, beta, 1e-8)
    g = torch.full((k,), 1.0 / 64, dtype=torch.float64)
    dX, dY, _, _ = OU.features_backward(X, Y, vx, vy, R, P, g, g if beta else 0 * g, 0.1, beta,
                                        1e-8)
    return [r, p if beta else 0 * r, dX, dY]


@pytest.mark.parametrize("beta", [1.0, 0.0], ids=["udtw", "soft_dtw"])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_cfg3_full_batch(dtype, beta):
    """B = 64, N = M = 1024, D = 16, gamma = 0.1: uDTW (beta = 1, loss
    mean(d + omega)) and soft-DTW (beta = 0, sigma = 1, loss mean(d)), the
    forward and backward launched on the whole batch."""
    torch.set_num_threads(min(16, torch.get_num_threads()))
    X, Y, sx, sy = _cfg3(beta)
    got = [t.detach()[:CFG3_CHECKED] for t in _cfg3_gpu(X, Y, sx, sy, beta, dtype)]
    want = _cfg3_oracle(X, Y, sx, sy, beta, CFG3_CHECKED)
    errs = [maxnorm_err(a, b) if b.abs().max() > 0 else a.abs().max().item()
            for a, b in zip(got, want)]
    print("\ncfg3 {} {}: max-normalised errors (d, omega, dX, dY) {}".format(
        "uDTW" if beta else "soft-DTW", dtype, ["%.2e" % e for e in errs]))
    if dtype == torch.float64:
        assert max(errs[:2]) < F64_TOL
        # The two float64 computations each carry their own rounding of the
        # DP at this scale (R reaches ~2.7e4 with gamma = 0.1): the float64
        # oracle is ~5e-10 from the extended-precision value
        # (tests/test_oracle_longdouble.py), and test_cfg3_float64_against_
        # extended_precision below bounds this kernel's own distance to it.
        assert max(errs[2:]) < 2e-9
    else:
        assert errs[0] < F32_VALUE_TOL
        assert errs[1] < 1e-4
        # The reference documents 1e-2 for its float32 kernel at N = 1000,
        # gamma = 0.1 (docs/limitations.md:31-36).
        assert max(errs[2:]) < CFG3_F32_GRAD_TOL


# float32 gradients at cfg3, relative to the largest entry: measured 1.1e-3
# (uDTW) and 1.3e-5 (soft-DTW) with R carried in double precision (5e-2 and
# 2.8e-2 with float32 R); the gate is about 3x the measured uDTW error.
CFG3_F32_GRAD_TOL = 3e-3


@pytest.mark.parametrize("beta", [1.0, 0.0], ids=["udtw", "soft_dtw"])
def test_cfg3_float64_against_extended_precision(beta):
    """Pair 0 of cfg3 in float64 on the GPU (launched with the full batch)
    against the same pair in 80-bit extended precision (oracle/udtw_ld.py):
    the kernel's gradients must be at least as close to the extended-precision
    value as the float64 oracle's (which follows the reference's algorithm)."""
    import numpy as np
    from oracle import udtw_ld
    X, Y, sx, sy = _cfg3(beta)
    got = [t.detach()[:1].double().cpu().numpy() for t in
           _cfg3_gpu(X, Y, sx, sy, beta, torch.float64)]
    vx, vy = (sx[0, :, 0] ** 2).numpy(), (sy[0, :, 0] ** 2).numpy()
    r, p, dX, dY, _, _ = udtw_ld.features_value_and_grads(
        X[0].numpy(), Y[0].numpy(), vx, vy, 0.1, beta, 1e-8, 1.0 / 64, (1.0 / 64) if beta else 0.0)
    ref = _cfg3_oracle(X, Y, sx, sy, beta, 1)

    def err(a, b):
        a, b = np.asarray(a, np.longdouble).ravel(), np.asarray(b, np.longdouble).ravel()
        return float(np.abs(a - b).max() / np.abs(b).max())
    hip = [err(got[2][0], dX), err(got[3][0], dY)]
    orc = [err(ref[2][0].numpy(), dX), err(ref[3][0].numpy(), dY)]
    print("\ncfg3 pair 0 {} float64 vs extended precision: HIP dX, dY {}, float64 oracle {}"
          .format("uDTW" if beta else "soft-DTW", ["%.2e" % e for e in hip],
                  ["%.2e" % e for e in orc]))
    assert err(got[0][0], r) < 1e-13
    assert max(hip) < max(2 * max(orc), 1e-10)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_cfg4_jeanie_features(dtype):
    q, s = make_inputs("cfg4", dtype=torch.float64)
    qq, ss = q.to(DEV, dtype).requires_grad_(True), s.to(DEV, dtype).requires_grad_(True)
    d = TF.jeanie(qq, ss, gamma=0.1, max_shift=1)
    d.mean().backward()
    qo, so = q.clone().requires_grad_(True), s.clone().requires_grad_(True)
    do = OJ.jeanie_from_cost(OJ.euclidean_cost(qo, so), gamma=0.1, max_shift=1)
    gq, gs = torch.autograd.grad(do.mean(), (qo, so))
    _check([d, d, qq.grad, ss.grad], [do, do, gq, gs], dtype, "cfg4")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_cfg5_jeanie_two_axes(dtype):
    (c,) = make_inputs("cfg5a", dtype=torch.float64)
    c5 = c.view(1024, 5, 5, 16, 16)
    x = c5.to(DEV, dtype).requires_grad_(True)
    d = TF.jeanie_from_cost(x, gamma=0.1, max_shift=1)
    d.mean().backward()
    out, R = OJ.forward(c5, 1, 1, 0.1)
    dC = OJ.backward(c5, R, torch.full((1024,), 1 / 1024, dtype=torch.float64), 1, 1, 0.1)
    _check([d, d, x.grad], [out, out, dC], dtype, "cfg5a")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_cfg5_fvm(dtype):
    (c,) = make_inputs("cfg5b", dtype=torch.float64)
    x = c.to(DEV, dtype).requires_grad_(True)
    d = TF.fvm_from_cost(x, gamma=0.1)
    d.mean().backward()
    want_d = OJ.fvm_from_cost(c, gamma=0.1)
    want_g = OJ.fvm_backward(c, torch.full((1024,), 1 / 1024, dtype=torch.float64), 0.1)
    _check([d, d, x.grad], [want_d, want_d, want_g], dtype, "cfg5b")


def test_cfg2_bitwise_deterministic():
    X, Y, sx, sy = make_inputs("cfg2", DEV)
    first = _udtw_gpu(X, Y, sx, sy, 1.0, 1.0, torch.float32)
    for _ in range(2):
        again = _udtw_gpu(X, Y, sx, sy, 1.0, 1.0, torch.float32)
        assert all(torch.equal(a, b) for a, b in zip(first, again))


def test_cfg5_bitwise_deterministic():
    (c,) = make_inputs("cfg5a", DEV)

    def run():
        x = c.view(1024, 5, 5, 16, 16).detach().requires_grad_(True)
        d = TF.jeanie_from_cost(x, gamma=0.1, max_shift=1)
        d.mean().backward()
        return d, x.grad
    first = run()
    assert all(torch.equal(a, b) for a, b in zip(run(), first))
