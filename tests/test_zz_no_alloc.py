"""The FVM backward that allocates nothing (``tw_fvm_cost_bwd_noalloc_*``,
scratch in a file-scope device array) against the one that takes a workspace
(``tw_fvm_cost_bwd_*``): bitwise the same gradients on two calls in a row, the
second with a smaller input (the array keeps the first call's contents). The
first call's sequences are longer than one group of rows, so its soft-DTW
backward also keeps hand-off records in the array."""

import pytest
import torch

from torchwarp_amd import _hip

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def _forward(c, gamma):
    B, K, T, U = c.shape
    temporal, R = c.new_empty(B, T * U), c.new_empty(B, T * U)
    out, scratch = c.new_empty(B), c.new_empty(B)
    _hip.call("tw_fvm_cost_fwd", c.dtype, c, B, K, T, U, gamma, temporal, R, out, scratch)
    return temporal, R


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_fvm_backward_equals_workspace_version(dtype):
    g = torch.Generator().manual_seed(17)
    for shape, gamma in (((2, 3, 600, 640), 0.3), ((8, 5, 16, 20), 0.1)):
        B, K, T, U = shape
        c = (4.0 * torch.rand(*shape, generator=g, dtype=torch.float64)).to("cuda", dtype)
        gout = torch.rand(B, generator=g, dtype=torch.float64).to("cuda", dtype)
        temporal, R = _forward(c, gamma)
        es = c.element_size()
        nws = -(-_hip.library().tw_fvm_workspace_bytes(B, K, T, U, es) // es)
        want, ws = torch.empty_like(c), c.new_empty(nws)
        _hip.call("tw_fvm_cost_bwd", dtype, c, temporal, R, gout, B, K, T, U, gamma, want, ws,
                  nws * es)
        got = torch.full_like(c, float("nan"))
        _hip.call("tw_fvm_cost_bwd_noalloc", dtype, c, temporal, R, gout, B, K, T, U, gamma, got)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), shape
