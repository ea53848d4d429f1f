"""ctypes binding of ``libtorchwarp_hip.so`` (C ABI in ``include/torchwarp_hip.h``).

Replaces the reference's JIT loader (``src/torchwarp/_cuda.py:29-73``): the
library is built ahead of time (``torchwarp_amd/build.py``) and loaded from
this package directory. There is no fallback: when the library or a ROCm
device is missing, every entry point raises. PyTorch provides device memory
and the current stream; the library launches its own kernels on that stream.
"""

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libtorchwarp_hip.so"

# argument codes: p pointer, i int, f real (float or double by suffix),
# z size_t, s stream
SIGNATURES = {
    "tw_udtw_cost_fwd": "ppiiiffpppps",
    "tw_udtw_cost_bwd": "ppppppiiiffipppzs",
    "tw_udtw_cost_tangent": "ppppppppiiiffpppppzs",
    "tw_udtw_feat_fwd": "ppppiiiiffffipppppzs",
    "tw_udtw_feat_bwd": "ppppppppiiiiffffiippppppzs",
    "tw_jeanie_cost_fwd": "piiiiiiiifpps",
    "tw_jeanie_cost_bwd": "ppppiiiiiiiifps",
    "tw_jeanie_feat_fwd": "ppiiiiiiiifippps",
    "tw_jeanie_feat_bwd": "ppppppiiiiiiiifippps",
    "tw_fvm_cost_fwd": "piiiifpppps",
    "tw_fvm_cost_bwd": "ppppiiiifppzs",
    "tw_fvm_cost_bwd_noalloc": "ppppiiiifps",
    "tw_pair_cost_fwd": "ppiiiiips",
    "tw_pair_cost_bwd": "ppppiiiiipps",
    "tw_rbf_cost_fwd": "ppiiiifps",
    "tw_rbf_cost_bwd": "pppiiiifpps",
}

# entry points that exist in float64 only
SIGNATURES_F64 = {
    "tw_optimal_path": "piiiiiipppps",
}

METRIC_RAW, METRIC_SQEUC, METRIC_EUC = 0, 1, 2

_lib = None
_error = None


def _ctype(code, real):
    return {"p": ctypes.c_void_p, "i": ctypes.c_int, "f": real, "z": ctypes.c_size_t,
            "s": ctypes.c_void_p}[code]


def _load():
    global _lib, _error
    if _lib is not None or _error is not None:
        return _lib
    if os.environ.get("TORCHWARP_NO_CUDA") == "1":
        _error = RuntimeError("disabled by TORCHWARP_NO_CUDA=1")
        return None
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        _error = RuntimeError("cannot load {} ({}); build it with "
                              "`python -m torchwarp_amd.build`".format(LIB_PATH, exc))
        return None
    lib.tw_last_error.restype = ctypes.c_char_p
    lib.tw_version.restype = ctypes.c_int
    lib.tw_udtw_feat_workspace_bytes.restype = ctypes.c_size_t
    lib.tw_udtw_feat_workspace_bytes.argtypes = [ctypes.c_int] * 5
    lib.tw_noalloc_scratch_bytes.restype = ctypes.c_size_t
    lib.tw_noalloc_scratch_bytes.argtypes = []
    lib.tw_fvm_workspace_bytes.restype = ctypes.c_size_t
    lib.tw_fvm_workspace_bytes.argtypes = [ctypes.c_int] * 5
    lib.tw_udtw_cost_workspace_bytes.restype = ctypes.c_size_t
    lib.tw_udtw_cost_workspace_bytes.argtypes = [ctypes.c_int] * 4
    lib.tw_udtw_feat_band_workspace_bytes.restype = ctypes.c_size_t
    lib.tw_udtw_feat_band_workspace_bytes.argtypes = [ctypes.c_int] * 4 + [ctypes.c_double,
                                                                           ctypes.c_int]
    lib.tw_udtw_cost_band_workspace_bytes.restype = ctypes.c_size_t
    lib.tw_udtw_cost_band_workspace_bytes.argtypes = [ctypes.c_int] * 3 + [ctypes.c_double,
                                                                           ctypes.c_int]
    lib.tw_udtw_tangent_workspace_bytes.restype = ctypes.c_size_t
    lib.tw_udtw_tangent_workspace_bytes.argtypes = [ctypes.c_int] * 5
    lib.tw_udtw_carry_bytes.restype = ctypes.c_size_t
    lib.tw_udtw_carry_bytes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_double, ctypes.c_int]
    lib.tw_async_status.restype = ctypes.c_int
    lib.tw_async_status.argtypes = [ctypes.c_int]
    lib.tw_test_set_wait.restype = None
    lib.tw_test_set_wait.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.tw_test_set_mw.restype = None
    lib.tw_test_set_mw.argtypes = [ctypes.c_int]
    for base, sig in SIGNATURES.items():
        for suffix, real in (("_f32", ctypes.c_float), ("_f64", ctypes.c_double)):
            fn = getattr(lib, base + suffix)
            fn.restype = ctypes.c_int
            fn.argtypes = [_ctype(c, real) for c in sig]
    for base, sig in SIGNATURES_F64.items():
        fn = getattr(lib, base + "_f64")
        fn.restype = ctypes.c_int
        fn.argtypes = [_ctype(c, ctypes.c_double) for c in sig]
    _lib = lib
    return lib


def library():
    """The loaded library; raises RuntimeError if it cannot be loaded."""
    lib = _load()
    if lib is None:
        raise _error
    return lib


def build_error():
    _load()
    return _error


def available():
    """True when the HIP library loads and a ROCm device is present."""
    return _load() is not None and torch.cuda.is_available()


_FNS = {}


def _entry(base, dtype):
    fn = _FNS.get((base, dtype))
    if fn is None:
        suffix = {torch.float32: "_f32", torch.float64: "_f64"}.get(dtype)
        if suffix is None:
            raise TypeError("torchwarp_amd computes in float32 or float64, got {}".format(dtype))
        fn = _FNS[(base, dtype)] = getattr(library(), base + suffix)
    return fn


def call(base, dtype, *args):
    """Call ``base``_f32/_f64 on the current stream of the first tensor's device.

    Kernels launch on the HIP device that is current during the call, so the
    tensors' device is made current when it is not already.
    """
    fn = _entry(base, dtype)
    dev = None
    cargs = []
    for a in args:
        if isinstance(a, torch.Tensor):
            if dev is None:
                dev = a.device.index
            cargs.append(a.data_ptr() if a.numel() else None)
        else:
            cargs.append(a)
    if torch._C._cuda_getDevice() == dev:
        rc = fn(*cargs, torch._C._cuda_getCurrentRawStream(dev))
    else:
        with torch.cuda.device(dev):
            rc = fn(*cargs, torch._C._cuda_getCurrentRawStream(dev))
    if rc != 0:
        raise RuntimeError("torchwarp_amd: " + _lib.tw_last_error().decode())
    if _CHECK_ASYNC:
        check_async_status(dev)


# TORCHWARP_CHECK_ASYNC=1: synchronise after every launch and raise at once if
# a bounded cross-workgroup wait gave up (a debugging mode, like a blocking
# launch mode; it cannot be used under stream capture).
_CHECK_ASYNC = os.environ.get("TORCHWARP_CHECK_ASYNC") == "1"


def check_async_status(device=None, clear=True):
    """Synchronise ``device`` (default: the current one) and raise RuntimeError
    if a uDTW sweep split over several workgroups per pair gave up waiting for
    a neighbouring workgroup's boundary row since the last check (that call's
    outputs are NaN). The status is sticky until checked; ``clear`` resets it."""
    lib = library()
    if device is None:
        dev = torch.cuda.current_device()
    elif isinstance(device, int):
        dev = device
    else:
        dev = torch.device(device).index
        dev = torch.cuda.current_device() if dev is None else dev
    with torch.cuda.device(dev):
        rc = lib.tw_async_status(1 if clear else 0)
    if rc != 0:
        raise RuntimeError("torchwarp_amd: " + lib.tw_last_error().decode())


def carry_cols(N, M, gamma, dtype):
    """Columns of the [B, cols] tensor (of ``dtype``) that holds the uDTW
    forward's R for the backward: N * M, or 2 * N * M for float32 when the
    kernels keep R in double precision (long sequences at a small gamma)."""
    es = 4 if dtype == torch.float32 else 8
    nbytes = library().tw_udtw_carry_bytes(1, N, M, float(gamma), es)
    return nbytes // es


def check_udtw_plane(N, M, gamma, dtype):
    """The kernels address one pair's N x M planes with 32-bit byte offsets;
    past that size raise ValueError, as the reference does for its kernels'
    size limit (udtw/_ops.py:45-50). There is no limit on the length itself."""
    es = 4 if dtype == torch.float32 else 8
    nbytes = max(carry_cols(N, M, gamma, dtype), N * M) * es
    if nbytes >= 1 << 31:
        raise ValueError(
            "uDTW: one pair's {} x {} dynamic-programming plane takes {} bytes; the HIP kernels "
            "handle planes below 2 GiB (2^29 cells in float32, 2^28 in float64). Shorten or "
            "downsample the sequences.".format(N, M, nbytes))


def udtw_workspace_elems(B, N, M, D, dtype=torch.float32, bandwidth=0.0):
    """Elements (of ``dtype``) of the workspace a feature-path uDTW backward
    needs: the squared-distance plane for D > 1 and, for sequences longer
    than one workgroup holds, the hand-off records between workgroups; with
    a band narrower than the grid, the B*N*M-element plane of the banded
    feature path (D = 1 included)."""
    es = 4 if dtype == torch.float32 else 8
    n = library().tw_udtw_feat_band_workspace_bytes(B, N, M, D, float(bandwidth or 0.0), es)
    return -(-n // es)


def udtw_feat_plane(B, N, M, D, dtype=torch.float32, bandwidth=0.0):
    """Whether a feature-path uDTW forward needs its B*N*M-element workspace
    plane: the squared distances (D > 1), or the banded path's cost and
    penalty (D = 1 with a band narrower than the grid)."""
    if D > 1:
        return True
    if not bandwidth or bandwidth <= 0:
        return False
    B, N, M, D = int(B), int(N), int(M), int(D)   # concrete sizes for the C query
    return udtw_workspace_elems(B, N, M, D, dtype, bandwidth) >= B * N * M


def udtw_cost_workspace_elems(B, N, M, dtype=torch.float32, bandwidth=0.0):
    """Elements (of ``dtype``) of the workspace a cost-path uDTW backward uses:
    the hand-off records between workgroups of long sequences, and with a band
    narrower than the grid the gradients in the banded sweep's layout (0 when
    neither applies)."""
    es = 4 if dtype == torch.float32 else 8
    lib = library()
    n = lib.tw_udtw_cost_band_workspace_bytes(B, N, M, float(bandwidth or 0.0), es)
    return -(-n // es)


def udtw_tangent_workspace_elems(B, N, M, has_penalty, dtype=torch.float32):
    """Elements (of ``dtype``) of the workspace of the second-order sweeps
    (``tw_udtw_cost_tangent``): the forward's R, P and their tangents, and for
    long sequences the diagonals the sweeps exchange."""
    es = 4 if dtype == torch.float32 else 8
    return -(-library().tw_udtw_tangent_workspace_bytes(B, N, M, int(bool(has_penalty)), es)
             // es)


def dense(dtype, *tensors, contiguous=True):
    """The tensors in ``dtype`` (and contiguous), converting only those that
    need it."""
    out = []
    for t in tensors:
        if t.dtype != dtype:
            t = t.to(dtype)
        if contiguous and not t.is_contiguous():
            t = t.contiguous()
        out.append(t)
    return out


def per_pair(*grads):
    """Per-pair gradient tensors [B] and their common element stride: a stride-0
    expansion (a mean's backward) is passed as is, anything else contiguous."""
    if all(g.dim() == 1 and g.stride(0) == 0 for g in grads):
        return grads, 0
    return tuple(g.contiguous() for g in grads), 1


def check_backend(backend):
    if backend not in ("auto", "cuda", "torch"):
        raise ValueError("backend must be 'auto', 'cuda' or 'torch'")


def require(t, backend, what):
    """Every computation runs on the HIP kernels; say so loudly otherwise."""
    check_backend(backend)
    if backend == "torch":
        raise ValueError(
            "{}: backend='torch' (the reference's portable PyTorch dynamic program) is not part "
            "of torchwarp_amd, which runs the HIP kernels only; use backend='auto' or "
            "'cuda'".format(what))
    if not t.is_cuda:
        raise RuntimeError(
            "{}: torchwarp_amd runs on ROCm GPUs only; move the inputs to a 'cuda' device "
            "(got a {} tensor)".format(what, t.device.type))
    if t.dtype not in (torch.float32, torch.float64):
        raise TypeError("{}: expected float32 or float64, got {}".format(what, t.dtype))
    library()
