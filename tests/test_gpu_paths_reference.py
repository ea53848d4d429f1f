"""torchwarp_amd.paths against the behaviours the reference pins for
``torchwarp.paths`` (its tests/test_paths.py:30-133), checked here through
this repository's own oracle (``oracle/brute.py``, ``oracle/paths.py``).

What is established, on CUDA tensors:
- at a tiny temperature the soft alignment's optimal path is a hard DTW path
  whose summed cost is the textbook DTW value, and its path matrix is a
  probability field that is 1 at both corners;
- uDTW / JEANIE / FVM alignments report the distances of the functional API;
- JEANIE paths change viewpoint by at most ``max_shift`` per step and start at
  ``start_view`` when one is given (which can only raise the distance);
- on grids small enough to enumerate, the path matrix, the distance and the
  optimal path equal the enumeration over every monotone path.
"""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF
from oracle import brute
from oracle.paths import optimal_3d
from torchwarp_amd import paths

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"
STEPS = {(1, 0), (0, 1), (1, 1)}


def _is_monotone_corner_path(p, T, U):
    cells = [tuple(c[:2]) for c in p]
    moves = {(b[0] - a[0], b[1] - a[1]) for a, b in zip(cells, cells[1:])}
    return cells[0] == (0, 0) and cells[-1] == (T - 1, U - 1) and moves <= STEPS


def test_hard_limit_of_soft_dtw_is_the_dtw_path():
    g = torch.Generator().manual_seed(11)
    cost = torch.rand(4, 8, 11, generator=g, dtype=torch.float64)
    al = paths.soft_dtw(cost.to(DEV), gamma=1e-3)
    pm = al.path_matrix.cpu()
    for b in range(cost.shape[0]):
        p = al.optimal_path[b]
        assert _is_monotone_corner_path(p, 8, 11)
        assert sum(cost[b, t, u].item() for t, u in p) == pytest.approx(
            brute.exact_dtw(cost[b]), abs=1e-9)
        # the hard path is the oracle's first-minimum backtrack, index for index
        assert [tuple(c) for c in p] == [c[:2] for c in optimal_3d(cost[b][None].numpy(), 0)]
        assert pm[b, 0, 0].item() == pytest.approx(1.0, abs=1e-6)
        assert pm[b, -1, -1].item() == pytest.approx(1.0, abs=1e-6)
        assert -1e-9 <= pm[b].min().item() and pm[b].max().item() <= 1.0 + 1e-6


def test_udtw_alignment_reports_the_module_outputs():
    g = torch.Generator().manual_seed(5)
    X = torch.randn(3, 6, 2, generator=g, dtype=torch.float64).to(DEV)
    Y = torch.randn(3, 10, 2, generator=g, dtype=torch.float64).to(DEV)
    sx = (0.5 + torch.rand(3, 6, 1, generator=g, dtype=torch.float64)).to(DEV)
    sy = (0.5 + torch.rand(3, 10, 1, generator=g, dtype=torch.float64)).to(DEV)
    al = paths.udtw(X, Y, sx, sy, gamma=0.2, beta=0.5)
    d, om = tw.UDTW(gamma=0.2, beta=0.5)(X, Y, sx, sy)
    torch.testing.assert_close(al.distance, d)
    torch.testing.assert_close(al.Omega, om)
    assert al.Sigma.shape == al.path_matrix.shape == (3, 6, 10)
    assert all(_is_monotone_corner_path(p, 6, 10) for p in al.optimal_path)


@pytest.mark.parametrize("max_shift", [1, 2])
def test_jeanie_and_fvm_alignments(max_shift):
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 6, 7, 3, generator=g, dtype=torch.float64).to(DEV)
    s = torch.randn(2, 9, 3, generator=g, dtype=torch.float64).to(DEV)
    cost = tw.euclidean_cost(q, s)
    al = paths.jeanie(q, s, gamma=0.1, max_shift=max_shift)
    torch.testing.assert_close(al.distance,
                               TF.jeanie_from_cost(cost, gamma=0.1, max_shift=max_shift))
    assert al.path_matrix.shape == (2, 6, 7, 9)
    for p in al.optimal_path:
        assert _is_monotone_corner_path(p, 7, 9)
        assert max(abs(b[2] - a[2]) for a, b in zip(p, p[1:])) <= max_shift

    pinned = paths.jeanie(q, s, gamma=0.1, max_shift=max_shift, start_view=2)
    assert {p[0][2] for p in pinned.optimal_path} == {2}
    # fewer admissible paths: the softmin over a subset is never smaller
    assert bool((pinned.distance >= al.distance - 1e-9).all())

    f = paths.fvm(q, s, gamma=0.1)
    torch.testing.assert_close(f.distance, TF.fvm_from_cost(cost, gamma=0.1))
    assert all(_is_monotone_corner_path(p, 7, 9) for p in f.optimal_path)

    per_view = paths.soft_dtw_per_view(q, s, gamma=0.1)
    assert len(per_view) == 6
    for k, v in enumerate(per_view):
        assert {c[2] for p in v.optimal_path for c in p} == {k}


@pytest.mark.parametrize("fn, args", [
    (paths.soft_dtw, ((4, 5),)),
    (paths.jeanie, ((5, 7, 4), (9, 4))),
    (paths.fvm, ((5, 7, 4), (9, 4))),
])
def test_inputs_without_a_batch_dimension_raise(fn, args):
    with pytest.raises(ValueError):
        fn(*[torch.randn(*shape, device=DEV) for shape in args])


@pytest.mark.parametrize("gamma", [0.1, 1.0])
@pytest.mark.parametrize("max_shift", [1, 2])
@pytest.mark.parametrize("start_view", [None, 1])
def test_jeanie_alignment_equals_path_enumeration(gamma, max_shift, start_view):
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 3, 4, 3, generator=g, dtype=torch.float64)
    s = torch.randn(1, 5, 3, generator=g, dtype=torch.float64)
    al = paths.jeanie(q.to(DEV), s.to(DEV), gamma=gamma, max_shift=max_shift,
                      start_view=start_view)
    cost = al.cost[0].cpu()
    every = brute.all_paths(3, 4, 5, max_shift)
    keep = [p for p in every if start_view is None or p[0][2] == start_view]
    w = torch.tensor([sum(cost[k, t, u].item() for t, u, k in p) for p in keep],
                     dtype=torch.float64)
    prob = torch.softmax(-w / gamma, 0)
    pm = torch.zeros_like(cost)
    for a, p in zip(prob.tolist(), keep):
        for t, u, k in p:
            pm[k, t, u] += a
    torch.testing.assert_close(al.path_matrix[0].cpu(), pm, atol=1e-9, rtol=0)
    assert al.distance[0].item() == pytest.approx(
        (-gamma * torch.logsumexp(-w / gamma, 0)).item(), rel=1e-12, abs=1e-12)
    assert [tuple(c) for c in al.optimal_path[0]] == keep[int(w.argmin())]
