"""The second-order sweeps' device code, run on the CPU against the oracle.

``tests/host/tangent_host.cpp`` calls the function the HIP kernel runs
(``tangent_pair`` of ``torchwarp_amd/csrc/udtw_tangent.hip``) with a
workgroup of CPU threads that meet at a barrier where the kernel has its
workgroup barrier, under AddressSanitizer. This checks every index the sweeps
use (inputs, the exchanged-diagonal ring, the skewed planes, the outputs of
every pair) and their arithmetic against ``oracle/udtw_tangent.py``, without
a GPU. The entry points ``tw_udtw_cost_tangent_*`` are switched off in the
library until the fault of their first GPU run is explained; this test keeps
the code they would run correct meanwhile.
"""

import os
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.udtw_tangent import dp_tangent

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="needs hipcc")


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    d = tmp_path_factory.mktemp("tangent_host")
    common = ["-O1", "-g", "-std=c++17", "-I" + str(ROOT / "include")]
    capi = d / "capi.o"
    subprocess.run([HIPCC, *common, "-c", str(ROOT / "torchwarp_amd/csrc/capi.cpp"), "-o",
                    str(capi)], check=True, capture_output=True)
    exe = d / "tangent_host"
    cmd = [HIPCC, "-x", "hip", "--offload-arch=gfx950", *common,
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Xarch_host", "-fsanitize=address", "-pthread",
           str(ROOT / "tests/host/tangent_host.cpp"), "-x", "none", str(capi), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def _rand(shape, seed, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return shift + scale * torch.rand(shape, generator=g, dtype=torch.float64)


CASES = [  # (B, N, M, gamma, bandwidth, penalty, threads)
    (3, 5, 7, 0.7, 0.0, True, 64),
    (2, 9, 5, 0.5, 0.0, True, 64),      # N > M
    (2, 14, 15, 1.0, 0.0, False, 64),   # no penalty
    (2, 10, 12, 0.3, 3.0, True, 64),    # band
    (1, 70, 75, 1.0, 0.0, True, 64),    # rows beyond the threads: row loop
    (2, 40, 45, 0.5, 6.0, True, 1),     # one thread: every row in turn
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}N{}M{}w{}{}t{}".format(
    c[0], c[1], c[2], c[4], "" if c[5] else "-nopen", c[6]))
def test_sweeps_on_the_cpu_match_oracle(harness, tmp_path, case):
    B, N, M, gamma, band, pen, threads = case
    C, Q = _rand((B, N, M), N, 3.0), _rand((B, N, M), N + 1, 0.5)
    tC, tQ = _rand((B, N, M), N + 2, 2.0, -1.0), _rand((B, N, M), N + 3, 2.0, -1.0)
    gr, gp, tgr, tgp = (_rand((B,), N + 4 + k, 2.0, -1.0) for k in range(4))
    if not pen:
        Q, tQ, gp, tgp = (torch.zeros_like(t) for t in (Q, tQ, gp, tgp))
    arrays = [C, Q, tC, tQ, gr, gp, tgr, tgp] if pen else [C, tC, gr, tgr]
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    np.concatenate([a.reshape(-1).numpy() for a in arrays]).tofile(fin)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1")
    r = subprocess.run([str(harness), str(B), str(N), str(M), str(int(pen)), repr(gamma),
                        repr(band), str(threads), str(fin), str(fout)],
                       capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    out = torch.from_numpy(np.fromfile(fout, dtype=np.float64))
    n = B * N * M
    got_c = out[:n].view(B, N, M)
    off = n
    if pen:
        got_q = out[off:off + n].view(B, N, M)
        off += n
    got_r = out[off:off + B]
    want = dp_tangent(C, Q, tC, tQ, gr, gp, tgr, tgp, gamma, band)
    rel = lambda a, b: ((a - b).abs().max() / b.abs().max()).item()
    assert rel(got_c, want[0]) < 1e-12
    assert (got_r - want[2]).abs().max().item() < 1e-12
    if pen:
        assert rel(got_q, want[1]) < 1e-12
        assert (out[off + B:off + 2 * B] - want[3]).abs().max().item() < 1e-12
