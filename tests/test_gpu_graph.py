"""Public-API steps captured as HIP graphs (torch.cuda.graph) replay the eager step.

Every entry point launches on the caller's stream, allocates nothing and
records no memset, so a forward + loss + backward through the public API
captures as is. Each case captures one step, then replays it three times with
eager steps and synchronisations in between; every replay's outputs and
gradients must be bitwise those of the eager step (the kernels are
deterministic). bench.py times the headline figure this way.
"""

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda"


def _inputs(shapes, seed):
    g = torch.Generator().manual_seed(seed)
    return [(0.5 + torch.rand(*s, generator=g)) if pos else torch.randn(*s, generator=g)
            for s, pos in shapes]


def _udtw(xs):
    d, p = tw.UDTW(gamma=0.7, beta=1.0)(*xs)
    return (d + p).mean()


CASES = {
    # name: (input shapes [(shape, positive)], loss of the leaves)
    "udtw_d1": ([((6, 40, 1), 0), ((6, 52, 1), 0), ((6, 40, 1), 1), ((6, 52, 1), 1)],
                _udtw),
    "udtw_d8_swap": ([((5, 33, 8), 0), ((5, 21, 8), 0), ((5, 33, 1), 1), ((5, 21, 1), 1)],
                     _udtw),
    # Sakoe-Chiba band: the reachability check is made from the shapes
    "udtw_band": ([((4, 30, 1), 0), ((4, 33, 1), 0), ((4, 30, 1), 1), ((4, 33, 1), 1)],
                  lambda xs: sum(tw.UDTW(gamma=0.7, beta=1.0, bandwidth=4)(*xs)).mean()),
    "soft_dtw": ([((4, 30, 3), 0), ((4, 25, 3), 0)],
                 lambda xs: tw.SoftDTW(gamma=0.5)(*xs).mean()),
    "udtw_from_cost": ([((3, 17, 23), 1), ((3, 17, 23), 1)],
                       lambda xs: sum(TF.udtw_from_cost(xs[0], xs[1], gamma=0.3)).sum()),
    # a band narrower than the grid: the banded sweep (band-compressed planes,
    # the zeroing workgroups in the backward's launch)
    "udtw_from_cost_band": ([((3, 40, 44), 1), ((3, 40, 44), 1)],
                            lambda xs: sum(TF.udtw_from_cost(xs[0], xs[1], gamma=0.3,
                                                             bandwidth=6.0)).sum()),
    # N > 256 and a small batch: several workgroups per pair in the forward
    # (sentinel fill kernel, polled hand-off between workgroups)
    "udtw_d1_groups": ([((2, 600, 1), 0), ((2, 620, 1), 0), ((2, 600, 1), 1),
                        ((2, 620, 1), 1)], _udtw),
    "udtw_from_cost_groups": ([((2, 300, 340), 1), ((2, 300, 340), 1)],
                              lambda xs: sum(TF.udtw_from_cost(xs[0], xs[1], gamma=0.3)).sum()),
    "jeanie_features": ([((7, 9, 8, 32), 0), ((7, 8, 32), 0)],
                        lambda xs: TF.jeanie(xs[0], xs[1], gamma=0.1, max_shift=1).mean()),
    "jeanie_cost_2axes": ([((6, 5, 5, 9, 7), 1)],
                          lambda xs: TF.jeanie_from_cost(xs[0], gamma=0.1, max_shift=1).mean()),
    "fvm_from_cost": ([((6, 25, 9, 7), 1)],
                      lambda xs: TF.fvm_from_cost(xs[0], gamma=0.1).mean()),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_graph_replay_matches_eager(name, dtype):
    shapes, loss_fn = CASES[name]
    base = [t.to(DEV, dtype) for t in _inputs(shapes, 11)]
    leaves = [t.clone().requires_grad_(True) for t in base]

    def step():
        for t in leaves:
            t.grad = None
        loss = loss_fn(leaves)
        loss.backward()
        return loss

    # eager reference on the same tensors
    want_loss = step().detach().clone()
    want = [t.grad.clone() for t in leaves]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        loss = step()
    grads = [t.grad for t in leaves]   # the graph's output buffers

    for r in range(3):
        # eager work between replays (its own kernels, allocations and syncs)
        for t in leaves:
            t.grad = None
        eager = loss_fn([t.detach().clone().requires_grad_(True) for t in base])
        torch.cuda.synchronize()
        assert torch.equal(eager.detach(), want_loss)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss.detach(), want_loss), (name, r)
        for k, (a, b) in enumerate(zip(grads, want)):
            assert torch.equal(a, b), (name, r, k, (a - b).abs().max().item())
