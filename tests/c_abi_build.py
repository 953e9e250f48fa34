"""Build recipe of tests/_build/c_abi_check, the native C++ caller of the C ABI
(tests/c_abi_check.cpp).  Test infrastructure: __graft_entry__.build() runs it
after building libkdecay.so, and the GPU test runs the binary."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCE = os.path.join(HERE, "c_abi_check.cpp")
BINARY = os.path.join(HERE, "_build", "c_abi_check")


def build(verbose: bool = False) -> str:
    from kilat_amd import _build

    os.makedirs(os.path.dirname(BINARY), exist_ok=True)
    libdir = os.path.dirname(_build.LIBRARY)
    cmd = [_build.hipcc(), "-O2", "-std=c++17", "-I", _build.INCLUDE, SOURCE, "-L", libdir, "-lkdecay",
           "-Wl,-rpath,$ORIGIN/../../kilat_amd", "-o", BINARY]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("building c_abi_check failed:\n" + proc.stdout)
    return BINARY
