"""The public call signatures equal the reference's (drop-in parity).

``golden/api_signatures.json`` holds the parameters (name, kind, default) of
every public function and module ``__init__`` / ``forward`` of the
reference's Python API, read from its source by ``golden/extract_signatures.py``.
Each must have the same parameters, in the same order and kind, with the
same defaults, in torchwarp_amd.
"""

import ast
import importlib
import inspect
import json
from pathlib import Path

import pytest

FIXTURE = Path(__file__).resolve().parent / "golden" / "api_signatures.json"
SIGS = json.loads(FIXTURE.read_text())
KIND = {inspect.Parameter.POSITIONAL_ONLY: "positional",
        inspect.Parameter.POSITIONAL_OR_KEYWORD: "positional",
        inspect.Parameter.VAR_POSITIONAL: "var_positional",
        inspect.Parameter.KEYWORD_ONLY: "keyword_only",
        inspect.Parameter.VAR_KEYWORD: "var_keyword"}


def _resolve(key):
    parts = key.split(".")
    for cut in range(len(parts) - 1, 0, -1):
        try:
            obj = importlib.import_module("torchwarp_amd." + ".".join(parts[:cut]))
        except ImportError:
            continue
        for attr in parts[cut:]:
            obj = getattr(obj, attr)
        return obj
    raise LookupError(key)


def _same_default(ours, ref_src):
    if ref_src is None:
        return ours is inspect.Parameter.empty
    try:
        return ours == ast.literal_eval(ref_src)
    except ValueError:
        return repr(ours) == ref_src


@pytest.mark.parametrize("key", sorted(SIGS))
def test_signature_matches_reference(key):
    ours = [p for p in inspect.signature(_resolve(key)).parameters.values() if p.name != "self"]
    ref = SIGS[key]
    assert [p.name for p in ours] == [r[0] for r in ref], key
    assert [KIND[p.kind] for p in ours] == [r[1] for r in ref], key
    for p, r in zip(ours, ref):
        assert _same_default(p.default, r[2]), (key, p.name, p.default, r[2])
