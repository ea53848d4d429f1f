"""torchwarp_amd: soft-DTW, uDTW, JEANIE and FVM on hand-written gfx950 (MI355X) HIP kernels.

A drop-in for torchwarp's public API (``src/torchwarp/__init__.py:1-21``):

    import torchwarp_amd as torchwarp
    import torchwarp_amd.functional as TF
"""

from . import _reference_ops, functional, paths  # noqa: F401  (registers the reference's op names)
from ._hip import check_async_status
from .jeanie import FVM, JEANIE, euclidean_cost, rbf_cost, squared_euclidean_cost
from .sdtw import SoftDTW
from .udtw import UDTW

__version__ = "0.1.0"

__all__ = [
    "UDTW", "SoftDTW", "JEANIE", "FVM", "euclidean_cost", "squared_euclidean_cost",
    "rbf_cost", "functional", "paths", "check_async_status",
]
