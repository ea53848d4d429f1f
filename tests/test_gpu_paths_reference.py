"""torchwarp_amd.paths on the cases of the reference's tests/test_paths.py:30-133.

Alignments (distance, path matrix, optimal path) on CUDA tensors: the hard
path at small gamma is the exact DTW path, the uDTW / JEANIE / FVM
alignments agree with the functional API, viewpoint steps respect
max_shift and start_view, and on tiny grids the path matrix and the
optimal path equal a brute-force enumeration of every monotone path.
"""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF
from torchwarp_amd import paths

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"


def exact_dtw(cost):
    T, U = cost.shape
    R = torch.full((T + 1, U + 1), float("inf"), dtype=cost.dtype)
    R[0, 0] = 0
    for t in range(1, T + 1):
        for u in range(1, U + 1):
            R[t, u] = cost[t - 1, u - 1] + min(R[t - 1, u], R[t, u - 1], R[t - 1, u - 1])
    return R[T, U]


def check_monotone(path, T, U):
    assert tuple(path[0][:2]) == (0, 0) and tuple(path[-1][:2]) == (T - 1, U - 1)
    for a, b in zip(path, path[1:]):
        assert (b[0] - a[0], b[1] - a[1]) in {(1, 0), (0, 1), (1, 1)}


def test_sdtw_hard_path_is_the_dtw_path():
    torch.manual_seed(0)
    cost = torch.rand(3, 9, 12, dtype=torch.float64)
    a = paths.soft_dtw(cost.to(DEV), gamma=1e-3)
    for b in range(3):
        check_monotone(a.optimal_path[b], 9, 12)
        along = sum(float(cost[b, t, u]) for t, u in a.optimal_path[b])
        assert along == pytest.approx(float(exact_dtw(cost[b])), abs=1e-9)
        assert float(a.path_matrix[b, 0, 0]) == pytest.approx(1.0, abs=1e-6)
        assert float(a.path_matrix[b, -1, -1]) == pytest.approx(1.0, abs=1e-6)
        assert float(a.path_matrix[b].min()) >= -1e-9
        assert float(a.path_matrix[b].max()) <= 1 + 1e-6


def test_udtw_alignment():
    torch.manual_seed(0)
    X = torch.randn(2, 7, 3, dtype=torch.float64, device=DEV)
    Y = torch.randn(2, 9, 3, dtype=torch.float64, device=DEV)
    sx = torch.rand(2, 7, 1, dtype=torch.float64, device=DEV) + 0.5
    sy = torch.rand(2, 9, 1, dtype=torch.float64, device=DEV) + 0.5
    a = paths.udtw(X, Y, sx, sy, gamma=0.1, beta=1.0)
    d, omega = tw.UDTW(gamma=0.1, beta=1.0)(X, Y, sx, sy)
    assert torch.allclose(a.distance, d) and torch.allclose(a.Omega, omega)
    assert a.path_matrix.shape == a.Sigma.shape == (2, 7, 9)
    for p in a.optimal_path:
        check_monotone(p, 7, 9)


@pytest.mark.parametrize("max_shift", [1, 2])
def test_jeanie_and_fvm_paths(max_shift):
    torch.manual_seed(0)
    q = torch.randn(2, 5, 8, 4, dtype=torch.float64, device=DEV)
    s = torch.randn(2, 10, 4, dtype=torch.float64, device=DEV)
    cost = tw.euclidean_cost(q, s)
    j = paths.jeanie(q, s, gamma=0.1, max_shift=max_shift)
    assert torch.allclose(j.distance, TF.jeanie_from_cost(cost, gamma=0.1, max_shift=max_shift))
    assert j.path_matrix.shape == (2, 5, 8, 10)
    for p in j.optimal_path:
        check_monotone(p, 8, 10)
        assert all(abs(b[2] - a[2]) <= max_shift for a, b in zip(p, p[1:]))
    k0 = 3
    js = paths.jeanie(q, s, gamma=0.1, max_shift=max_shift, start_view=k0)
    assert all(p[0][2] == k0 for p in js.optimal_path)
    assert torch.all(js.distance >= j.distance - 1e-9)
    f = paths.fvm(q, s, gamma=0.1)
    assert torch.allclose(f.distance, TF.fvm_from_cost(cost, gamma=0.1))
    for p in f.optimal_path:
        check_monotone(p, 8, 10)
    views = paths.soft_dtw_per_view(q, s, gamma=0.1)
    assert len(views) == 5
    for k, v in enumerate(views):
        assert all(c[2] == k for p in v.optimal_path for c in p)


def test_unbatched_inputs_raise():
    with pytest.raises(ValueError):
        paths.soft_dtw(torch.rand(4, 5, device=DEV))
    with pytest.raises(ValueError):
        paths.jeanie(torch.randn(5, 7, 4, device=DEV), torch.randn(9, 4, device=DEV))
    with pytest.raises(ValueError):
        paths.fvm(torch.randn(5, 7, 4, device=DEV), torch.randn(9, 4, device=DEV))


def all_paths(K, T, U, max_shift):
    out = []

    def rec(k, t, u, p):
        if (t, u) == (T - 1, U - 1):
            out.append(p)
            return
        for dt, du in ((1, 0), (0, 1), (1, 1)):
            for dk in range(-max_shift, max_shift + 1):
                if t + dt < T and u + du < U and 0 <= k + dk < K:
                    rec(k + dk, t + dt, u + du, p + [(t + dt, u + du, k + dk)])
    for k in range(K):
        rec(k, 0, 0, [(0, 0, k)])
    return out


@pytest.mark.parametrize("gamma", [0.1, 1.0])
@pytest.mark.parametrize("max_shift", [1, 2])
def test_paths_match_enumeration(gamma, max_shift):
    torch.manual_seed(1)
    q = torch.randn(1, 3, 4, 3, dtype=torch.float64)
    s = torch.randn(1, 5, 3, dtype=torch.float64)
    for start in (None, 1):
        j = paths.jeanie(q.to(DEV), s.to(DEV), gamma=gamma, max_shift=max_shift, start_view=start)
        P = [p for p in all_paths(3, 4, 5, max_shift) if start is None or p[0][2] == start]
        cl = j.cost[0].cpu().tolist()   # plain floats: the enumeration is large
        w = torch.tensor([sum(cl[k][t][u] for t, u, k in p) for p in P], dtype=torch.float64)
        weights = torch.softmax(-w / gamma, 0).tolist()
        pm = [[[0.0] * 5 for _ in range(4)] for _ in range(3)]
        for a, p in zip(weights, P):
            for t, u, k in p:
                pm[k][t][u] += a
        assert torch.allclose(j.path_matrix[0].cpu(), torch.tensor(pm, dtype=torch.float64),
                              atol=1e-9)
        assert float(j.distance[0]) == pytest.approx(float(-gamma * torch.logsumexp(-w / gamma, 0)))
        assert [tuple(c) for c in j.optimal_path[0]] == P[int(w.argmin())]
