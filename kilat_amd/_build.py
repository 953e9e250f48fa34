"""Build recipe of ``libkdecay.so``: one hipcc invocation for gfx950.

Run ``python -m kilat_amd._build`` (or ``__graft_entry__.build()``).  The
library is written in-tree next to this file, where ``kilat_amd._lib`` loads it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCE = os.path.join(HERE, "csrc", "kdecay.hip")
INCLUDE = os.path.join(ROOT, "include")
LIBRARY = os.path.join(HERE, "libkdecay.so")

# -packed-fp32-ops: no v_pk_*_f32 in the device code.
# -mcode-object-version=5: loadable by torch's bundled ROCm 7.0 runtime.
# No fast-math: fp32 division stays correctly rounded (hipcc's default), and
# the source turns fp contraction off itself.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libkdecay.so)")
    return path


def build_library(verbose: bool = False) -> str:
    """Compile csrc/kdecay.hip into libkdecay.so; returns the library path."""
    tmp = LIBRARY + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, SOURCE, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and says
    # so; that line is expected and not shown.
    lines = [l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
