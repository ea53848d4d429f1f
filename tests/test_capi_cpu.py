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
    assert len(names) == 34
    for name in names:
        assert hasattr(lib, name), name
    assert lib.tw_version() == 1


def test_binding_covers_every_entry_point():
    bound = {"tw_version", "tw_last_error", "tw_udtw_feat_workspace_bytes", "tw_async_status",
             "tw_test_set_wait"}
    for base in _hip.SIGNATURES:
        bound |= {base + "_f32", base + "_f64"}
    bound |= {base + "_f64" for base in _hip.SIGNATURES_F64}
    assert set(_declared()) == bound


def test_workspace_query_is_host_only():
    lib = _hip.library()
    assert lib.tw_udtw_feat_workspace_bytes(2, 3, 4, 1, 4) == 0
    assert lib.tw_udtw_feat_workspace_bytes(2, 3, 4, 5, 4) == 2 * 3 * 4 * 4


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
