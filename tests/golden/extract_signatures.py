"""Write api_signatures.json: the public call signatures of the reference's
Python API, read from its source with ``ast`` (nothing of it is imported or
run). Run from the repository root where /root/reference exists:

    python tests/golden/extract_signatures.py /root/reference/src/torchwarp

Each entry maps "module.name" (for classes, "module.Class.__init__" and
"module.Class.forward") to its parameters: [name, kind, default source].
"""

import ast
import json
import sys
from pathlib import Path

MODULES = ["functional", "sdtw", "paths", "udtw.functional", "udtw.module",
           "jeanie.functional", "jeanie.fvm", "jeanie.distances", "jeanie.module"]


def _params(fn):
    a = fn.args
    out = []
    pos = a.posonlyargs + a.args
    defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
    for p, d in zip(pos, defaults):
        if p.arg == "self":
            continue
        out.append([p.arg, "positional", None if d is None else ast.unparse(d)])
    if a.vararg:
        out.append([a.vararg.arg, "var_positional", None])
    for p, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append([p.arg, "keyword_only", None if d is None else ast.unparse(d)])
    if a.kwarg:
        out.append([a.kwarg.arg, "var_keyword", None])
    return out


def main(root):
    root = Path(root)
    sigs = {}
    for mod in MODULES:
        tree = ast.parse((root / (mod.replace(".", "/") + ".py")).read_text())
        for node in tree.body:
            if isinstance(node, ast.FunctionDef) and not node.name.startswith("_"):
                sigs["{}.{}".format(mod, node.name)] = _params(node)
            elif isinstance(node, ast.ClassDef) and not node.name.startswith("_"):
                for item in node.body:
                    if isinstance(item, ast.FunctionDef) and item.name in ("__init__", "forward"):
                        sigs["{}.{}.{}".format(mod, node.name, item.name)] = _params(item)
    out = Path(__file__).resolve().parent / "api_signatures.json"
    out.write_text(json.dumps(sigs, indent=1, sort_keys=True) + "\n")
    print("wrote", out, len(sigs), "signatures")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/torchwarp")
