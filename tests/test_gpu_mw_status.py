"""A bounded cross-workgroup wait that runs out is reported, not silent.

The uDTW forward with several workgroups per pair hands each group's last row
to the next group and polls for it with a bounded loop. The test hook
``tw_test_set_wait`` (set from the host) shortens the poll to a few rounds and
keeps the producing group from storing that row at all, so the consumer's
wait runs out while every kernel still runs to its end. The call's outputs
are NaN (the pre-filled sentinel), ``check_async_status`` raises once, and the
next call, with the hook off, is correct again.
"""

import pytest
import torch

from oracle import udtw as OU
import torchwarp_amd as tw
from torchwarp_amd import _hip

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def _inputs():
    g = torch.Generator().manual_seed(31)
    # 500 rows, one pair: two workgroups of 256 rows, one hand-off (one row
    # per thread in both precisions)
    X = torch.randn(1, 500, 1, generator=g, dtype=torch.float64)
    Y = torch.randn(1, 520, 1, generator=g, dtype=torch.float64)
    sx = 0.5 + torch.rand(1, 500, 1, generator=g, dtype=torch.float64)
    sy = 0.5 + torch.rand(1, 520, 1, generator=g, dtype=torch.float64)
    return X, Y, sx, sy


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_wait_that_gives_up_is_reported(dtype):
    lib = _hip.library()
    tw.check_async_status()   # start from a clear status word
    X, Y, sx, sy = _inputs()
    xs = [t.to("cuda", dtype) for t in (X, Y, sx, sy)]
    m = tw.UDTW(gamma=1.0, beta=1.0)
    lib.tw_test_set_wait(4, 1)
    try:
        d, p = m(*xs)
        torch.cuda.synchronize()
    finally:
        lib.tw_test_set_wait(0, 0)
    assert torch.isnan(d).all() and torch.isnan(p).all()   # the sentinel, passed through
    with pytest.raises(RuntimeError, match="gave up waiting"):
        tw.check_async_status()
    tw.check_async_status()   # cleared by the check that raised

    d, p = m(*xs)
    rd, rp = OU.udtw(X, Y, sx, sy, gamma=1.0, beta=1.0)
    tol = 1e-10 if dtype == torch.float64 else 1e-5
    torch.testing.assert_close(d.double().cpu(), rd, rtol=tol, atol=tol * rd.abs().max().item())
    torch.testing.assert_close(p.double().cpu(), rp, rtol=tol, atol=tol * rp.abs().max().item())
    tw.check_async_status()
