"""Golden fixtures: inputs and outputs of the official uDTW / JEANIE code (float64).

``golden/reference_cases.pt`` is the reference's ``tests/golden/reference.pt``
copied as data by ``golden/extract.py``. Case keys are ``name|param=value|...``
with parameters sorted by name; the case-list constants below are the grids
the reference's generator used (``tests/golden.py:19-56``), needed to address
the stored cases.
"""

from pathlib import Path

import torch

PATH = Path(__file__).resolve().parent / "golden" / "reference_cases.pt"

UDTW_SHAPES = [(1, 1), (1, 6), (6, 1), (5, 8), (8, 5), (9, 9)]
GAMMAS = [0.01, 0.1, 1.0]
UDTW_BANDS = [(9, 9, 1), (9, 9, 2), (6, 10, 4), (10, 6, 4.5), (7, 7, 0)]
UDTW_BETAS = [0.0, 1.0, 3.0]
UDTW_MAML = [(False, None), (True, None), (False, 2)]
SDTW_SHAPES = [(1, 1), (1, 6), (6, 1), (5, 7), (8, 4), (9, 9)]
JEANIE_1D_SHAPES = [(1, 4, 5), (5, 6, 7), (5, 8, 5), (3, 1, 4)]
JEANIE_1D_SHIFTS = [0, 1, 2, 7]
JEANIE_2D_SHAPES = [(3, 3, 5, 6), (2, 4, 6, 4), (1, 3, 4, 4)]
JEANIE_2D_SHIFTS = [(0, 0), (1, 1), (1, 0), (2, 1)]
FVM_CASES = [
    ("fvm_query_only_1d", (4, 5, 6)),
    ("fvm_query_only_2d", (3, 3, 5, 6)),
    ("fvm_1d_from_cost", (3, 4, 6, 5)),
    ("fvm_2d_from_cost", (2, 2, 3, 2, 5, 6)),
]
DISTANCES = ["euclidean_cost", "squared_euclidean_cost", "rbf_cost"]
METRICS = ["euclidean", "sqeuclidean", "rbf"]
FEATURES_1D = [(5, 6, 8, 1), (3, 9, 4, 2), (1, 5, 5, 0)]
ACCUMULATOR_COST = [(4, 5, 7, 1), (3, 7, 4, 2), (1, 4, 4, 0)]
SECOND_ORDER = ["jeanie_cost", "jeanie_features", "fvm", "soft_dtw"]
UDTW_LARGE = [(2, 40, 50)]
LARGE_COST = [
    ("soft_dtw", (60, 70), None),
    ("jeanie_1d_from_cost", (5, 30, 40), 2),
    ("jeanie_1d_from_cost", (4, 35, 20), 1),
    ("jeanie_2d_from_cost", (3, 3, 20, 25), (1, 1)),
    ("fvm_query_only_1d", (5, 40, 50), None),
    ("fvm_query_only_2d", (2, 3, 30, 35), None),
]


def key(name, /, **params):
    return name + "".join("|{}={!r}".format(k, params[k]) for k in sorted(params))


_DATA = None


def golden(name, /, **params):
    """The stored inputs and official outputs of one case (dict of tensors)."""
    global _DATA
    if _DATA is None:
        _DATA = torch.load(PATH, weights_only=True)
    return _DATA[key(name, **params)]


def all_keys():
    golden("udtw.softmin")
    return list(_DATA)
