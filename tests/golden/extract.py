"""Write tests/golden/reference_cases.pt from the reference's golden file.

The reference ships ``tests/golden/reference.pt``: inputs and outputs of the
official uDTW / JEANIE implementations (float64, 147 cases, MIT licence).
This script copies that data -- tensors only, loaded with
``weights_only=True`` -- into a fixture this repository owns, together with
the case-list constants the reference's tests use (``tests/golden.py:19-56``),
so the tests never read ``/root/reference`` at run time.

Run once in the build container (where ``/root/reference`` exists):

    python tests/golden/extract.py
"""

from pathlib import Path

import torch

SRC = Path("/root/reference/tests/golden/reference.pt")
DST = Path(__file__).resolve().parent / "reference_cases.pt"


def _dense(x):
    if isinstance(x, torch.Tensor):
        return x.detach().clone().contiguous()
    if isinstance(x, (list, tuple)):
        return [_dense(y) for y in x]
    if isinstance(x, dict):
        return {k: _dense(v) for k, v in x.items()}
    raise TypeError(type(x))


def main():
    data = torch.load(SRC, weights_only=True)
    out = {k: _dense(v) for k, v in data.items()}
    torch.save(out, DST)
    print("wrote {} cases to {} ({:.0f} KiB)".format(len(out), DST, DST.stat().st_size / 1024))


if __name__ == "__main__":
    main()
