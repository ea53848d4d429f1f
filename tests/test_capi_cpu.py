"""CPU checks of the drop-in boundary: the C-ABI library loads, exports every
symbol ``include/torchwarp_hip.h`` declares, and the host layer validates
arguments (and refuses CPU execution) the way the reference does. No GPU
compute is called here."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import torchwarp_amd as tw
import torchwarp_amd.functional as TF
from torchwarp_amd import _hip

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "torchwarp_hip.h").read_text()
    return sorted(set(re.findall(r"\b(tw_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    names = _declared()
    assert len(names) == 46
    for name in names:
        assert hasattr(lib, name), name
    assert lib.tw_version() == 1


def test_binding_covers_every_entry_point():
    bound = {"tw_version", "tw_last_error", "tw_udtw_feat_workspace_bytes", "tw_async_status",
             "tw_test_set_wait", "tw_udtw_carry_bytes",
             "tw_udtw_cost_workspace_bytes", "tw_udtw_cost_band_workspace_bytes",
             "tw_udtw_feat_band_workspace_bytes",
             "tw_test_set_mw", "tw_fvm_workspace_bytes",
             "tw_noalloc_scratch_bytes", "tw_udtw_tangent_workspace_bytes"}
    for base in _hip.SIGNATURES:
        bound |= {base + "_f32", base + "_f64"}
    bound |= {base + "_f64" for base in _hip.SIGNATURES_F64}
    assert set(_declared()) == bound


def test_workspace_query_is_host_only():
    lib = _hip.library()
    # second-order sweeps: R, P and their tangents (4 planes; 2 without a
    # penalty), plus the exchanged diagonals (3 x 8 values per row; 3 x 4)
    # when they do not fit in the LDS
    assert lib.tw_udtw_tangent_workspace_bytes(2, 3, 4, 1, 8) == 2 * 4 * 3 * 4 * 8
    assert lib.tw_udtw_tangent_workspace_bytes(2, 3, 4, 0, 4) == 2 * 2 * 3 * 4 * 4
    assert lib.tw_udtw_tangent_workspace_bytes(1, 3000, 3100, 1, 8) == \
        (4 * 3000 * 3100 + 24 * 3000) * 8
    assert lib.tw_udtw_tangent_workspace_bytes(0, 3, 4, 1, 8) == 0
    assert lib.tw_udtw_feat_workspace_bytes(2, 3, 4, 1, 4) == 0
    assert lib.tw_udtw_feat_workspace_bytes(2, 3, 4, 5, 4) == 2 * 3 * 4 * 4
    # past 1024 rows (float; 512 in double) the backward runs ceil(N / 256)
    # workgroups per pair and hands boundary records (4 float / 6 double words
    # of 8 bytes per column) across the G - 1 group boundaries
    assert lib.tw_udtw_feat_workspace_bytes(1, 2000, 2100, 1, 4) == 7 * 2100 * 4 * 8
    assert lib.tw_udtw_feat_workspace_bytes(2, 2000, 2100, 5, 4) == \
        2 * 2000 * 2100 * 4 + 2 * 7 * 2100 * 4 * 8
    assert lib.tw_udtw_feat_workspace_bytes(1, 600, 700, 1, 8) == 2 * 700 * 6 * 8
    # a band narrower than the grid: the banded feature path's plane of
    # B*N*M elements, D = 1 included; otherwise the unbanded size
    assert lib.tw_udtw_feat_band_workspace_bytes(2, 300, 310, 1, 30.0, 4) == 2 * 300 * 310 * 4
    assert lib.tw_udtw_feat_band_workspace_bytes(2, 300, 310, 5, 30.0, 8) == 2 * 300 * 310 * 8
    plain = lib.tw_udtw_feat_workspace_bytes(2, 300, 310, 1, 4)
    assert lib.tw_udtw_feat_band_workspace_bytes(2, 300, 310, 1, 0.0, 4) == plain
    assert lib.tw_udtw_feat_band_workspace_bytes(2, 300, 310, 1, 299.0, 4) == plain
    assert lib.tw_udtw_feat_band_workspace_bytes(1, 2000, 2100, 1, 0.0, 4) == 7 * 2100 * 4 * 8
    assert lib.tw_udtw_cost_workspace_bytes(3, 1025, 1100, 4) == 3 * 4 * 1100 * 4 * 8
    assert lib.tw_udtw_cost_workspace_bytes(3, 1100, 1025, 4) == 3 * 4 * 1100 * 4 * 8
    # up to 1024 rows, pairs split over workgroups only when the batch has
    # fewer pairs than the device has CUs (256 assumed without a device)
    assert lib.tw_udtw_cost_workspace_bytes(3, 1024, 1100, 4) == 3 * 3 * 1100 * 4 * 8
    assert lib.tw_udtw_cost_workspace_bytes(300, 1024, 1100, 4) == 0
    assert lib.tw_udtw_cost_workspace_bytes(3, 256, 1100, 4) == 0


def test_cpu_tensors_fail_loudly():
    X, Y = torch.rand(2, 4, 1), torch.rand(2, 5, 1)
    S1, S2 = torch.ones(2, 4, 1), torch.ones(2, 5, 1)
    with pytest.raises(RuntimeError, match="ROCm"):
        tw.UDTW()(X, Y, S1, S2)
    with pytest.raises(RuntimeError, match="ROCm"):
        TF.jeanie_from_cost(torch.rand(1, 2, 4, 5))
    with pytest.raises(RuntimeError, match="ROCm"):
        TF.fvm_from_cost(torch.rand(1, 2, 4, 5))
    with pytest.raises(ValueError, match="backend='torch'"):
        TF.soft_dtw_from_cost(torch.rand(1, 4, 5), backend="torch")
    with pytest.raises(RuntimeError, match="ROCm"):
        tw.paths.optimal_path(torch.rand(1, 4, 5))


def test_udtw_input_validation():
    X, Y = torch.rand(2, 4, 5), torch.rand(2, 5, 5)
    SX, SY = torch.ones(2, 4, 1), torch.ones(2, 5, 1)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.0)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1, beta=-1.0)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1)(X[0], Y, SX, SY)
    with pytest.raises(ValueError):
        tw.UDTW(gamma=0.1, backend="nope")
    with pytest.raises(TypeError):
        TF.udtw(X, Y, SX, SY, 0.1, 1.0)
    with pytest.raises(ValueError):
        TF.udtw_from_cost(torch.rand(3, 4), torch.rand(3, 4))
    with pytest.raises(ValueError):
        TF.udtw(X, Y, SX, SY, bandwidth=-1)


def test_jeanie_input_validation():
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(torch.rand(4, 5), gamma=0.1)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(torch.rand(2, 4, 5), gamma=0.1)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(torch.rand(1, 2, 4, 5), gamma=0.0)
    with pytest.raises(ValueError):
        TF.jeanie_from_cost(torch.rand(1, 2, 4, 5), gamma=0.1, max_shift=-1)
    with pytest.raises(ValueError):
        TF.jeanie(torch.rand(2, 4, 3), torch.rand(5, 3))
    with pytest.raises(TypeError):
        TF.soft_dtw_from_cost(torch.ones(1, 3, 3, dtype=torch.int64))
    with pytest.raises(ValueError):
        TF.soft_dtw_from_cost(torch.rand(3, 3))
    with pytest.raises(ValueError):
        TF.fvm_from_cost(torch.rand(4, 5, 6))
    with pytest.raises(TypeError):
        TF.jeanie_from_cost(torch.rand(1, 2, 4, 5), 0.1)
    with pytest.raises(ValueError):
        tw.JEANIE(gamma=0.1, max_shift=(1, 1))(torch.rand(1, 2, 3, 4), torch.rand(1, 5, 4))


def test_exports_match_reference_surface():
    for name in ("UDTW", "SoftDTW", "JEANIE", "FVM", "euclidean_cost", "squared_euclidean_cost",
                 "rbf_cost", "functional"):
        assert hasattr(tw, name), name
    for name in ("udtw", "udtw_from_cost", "pairwise_matrices", "UDTWOutput", "soft_dtw",
                 "soft_dtw_from_cost", "jeanie", "jeanie_from_cost", "fvm", "fvm_from_cost",
                 "softmin", "softmin_weights", "euclidean_cost", "squared_euclidean_cost",
                 "rbf_cost"):
        assert hasattr(TF, name), name
    assert repr(tw.JEANIE(gamma=0.1, max_shift=(1, 1))).count("max_shift=(1, 1)") == 1


def _declared_arities():
    """name -> number of parameters, from the header's declarations."""
    text = (ROOT / "include" / "torchwarp_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(tw_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_signatures_match_the_header():
    """The ctypes argument codes (torchwarp_amd/_hip.py) have exactly as many
    entries as each declaration has parameters (the stream included)."""
    ar = _declared_arities()
    for base, sig in _hip.SIGNATURES.items():
        for suffix in ("_f32", "_f64"):
            assert ar[base + suffix] == len(sig), (base + suffix, ar[base + suffix], sig)
    for base, sig in _hip.SIGNATURES_F64.items():
        assert ar[base + "_f64"] == len(sig), base


def test_invalid_arguments_are_rejected_before_any_launch():
    """Argument errors return TW_EINVAL with a message and launch nothing, so
    they can be checked without a GPU."""
    lib = _hip.library()
    f = lib.tw_rbf_cost_fwd_f32
    assert f(None, None, 1, 2, 3, 4, -1.0, None, None) == 1
    assert b"sigma" in lib.tw_last_error()
    g = lib.tw_pair_cost_fwd_f32
    assert g(None, None, 1, 0, 3, 4, 1, None, None) == 1
    assert b"bad sizes" in lib.tw_last_error()
    h = lib.tw_rbf_cost_bwd_f64
    assert h(None, None, None, 2, -1, 3, 4, 0.5, None, None, None) == 1


def test_carry_bytes_query():
    """R is carried in the compute type, except float32 calls on long
    sequences at a small gamma, which keep R in double precision."""
    lib = _hip.library()
    q = lib.tw_udtw_carry_bytes
    assert q(256, 140, 140, 1.0, 4) == 256 * 140 * 140 * 4        # cfg2: float32 R
    assert q(64, 1024, 1024, 0.1, 4) == 64 * 1024 * 1024 * 8      # cfg3: double R
    assert q(64, 1024, 1024, 0.1, 8) == 64 * 1024 * 1024 * 8      # float64 anyway
    assert q(1, 2000, 2000, 0.1, 4) == 2000 * 2000 * 8            # several workgroups per pair
    assert q(1, 2000, 2000, 1.0, 4) == 2000 * 2000 * 8
    assert q(1, 700, 700, 1.0, 4) == 700 * 700 * 4               # scale 2016: float32 R
    assert q(1, 720, 720, 1.0, 4) == 720 * 720 * 8               # scale 2076: double R
    assert q(0, 5, 5, 1.0, 4) == 0
    assert _hip.carry_cols(1024, 1024, 0.1, torch.float32) == 2 * 1024 * 1024
    assert _hip.carry_cols(140, 140, 1.0, torch.float32) == 140 * 140


def test_noalloc_entry_rejects_sizes_past_its_scratch():
    """The FVM backward without allocation checks its fixed scratch before any
    launch: 4096 pairs of 64 x 64 in float64 need 128 MiB of it."""
    lib = _hip.library()
    assert lib.tw_noalloc_scratch_bytes() == 16 << 20
    rc = lib.tw_fvm_cost_bwd_noalloc_f64(None, None, None, None, 4096, 5, 64, 64, 0.1, None, None)
    assert rc == 3   # TW_ESIZE
    assert b"scratch" in lib.tw_last_error()
    assert lib.tw_fvm_cost_bwd_noalloc_f32(None, None, None, None, 0, 5, 6, 7, 0.1, None,
                                           None) == 0   # empty batch: no-op
