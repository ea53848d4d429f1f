"""Build the gfx950 HIP library ``torchwarp_amd/libtorchwarp_hip.so`` in-tree.

    python -m torchwarp_amd.build          # or __graft_entry__.build()

Every ``csrc/*.hip`` / ``csrc/*.cpp`` is compiled with hipcc for gfx950 in
parallel, then linked into one shared library exporting the C ABI declared
in ``include/torchwarp_hip.h``. Objects go to ``_build/`` (not committed).
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libtorchwarp_hip.so"
BUILD = ROOT / "_build"
ARCH = os.environ.get("TORCHWARP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
COMMON = [
    "--offload-arch=" + ARCH,
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-command-line-argument",
    # packed FP32 (v_pk_*_f32) stays off in every device pass
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + str(ROOT / "include"),
]


# Sources compiled once per set of defines (one object each): the uDTW sweep
# launchers per (type, direction, cost source), so their kernels build in
# parallel.
VARIANTS = {
    "udtw_sweep.hip": [
        {"TW_SWEEP_T": t, "TW_SWEEP_BWD": bwd, "TW_SWEEP_SRC": src}
        for t in ("float", "double") for bwd in ("0", "1") for src in ("0", "1", "2")
    ],
}


def _units():
    """(source, defines, object name) of every compilation unit."""
    units = []
    for src in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp")):
        for k, defs in enumerate(VARIANTS.get(src.name, [None])):
            stem = src.stem if defs is None else "{}_{}".format(src.stem, k)
            units.append((src, defs or {}, stem))
    # longest first: the double-precision sweeps dominate the build
    units.sort(key=lambda u: (u[1].get("TW_SWEEP_T") != "double", u[2]))
    return units


def _compile(unit):
    src, defs, stem = unit
    obj = BUILD / (stem + ".o")
    cmd = [HIPCC] + COMMON + ["-D{}={}".format(k, v) for k, v in defs.items()]
    cmd += ["-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, "-O2", "-fPIC", "-std=c++17", "-I" + str(ROOT / "include"),
               "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the device-only feature
    noise = ("packed-fp32-ops", "is not a recognized feature", "warning generated",
             "warnings generated")
    msg = "\n".join(line for line in (r.stdout + r.stderr).splitlines()
                    if line.strip() and not any(n in line for n in noise))
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on {}:\n{}".format(src.name, msg))
    return obj, msg


def build(verbose=False):
    """Compile every source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    units = _units()
    jobs = min(len(units), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        results = list(ex.map(_compile, units))
    for obj, msg in results:
        if verbose and msg:
            print(msg)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-o", str(tmp)] + [str(o) for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
