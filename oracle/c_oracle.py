"""Build and ctypes binding of oracle/decay_oracle.c — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__ and bench.py's cpu_baseline leg use it, as a
checker or the timed CPU baseline.  Built with gcc into oracle/_build/.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "decay_oracle.c")
LIBRARY = os.path.join(HERE, "_build", "libdecay_oracle.so")

# -ffp-contract=off: every multiply and add rounds on its own, as torch's
# separate ops do.  No -ffast-math.  x86-64 gcc uses SSE, so float math is
# evaluated in float (FLT_EVAL_METHOD 0).
GCC_CMD = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math"]

_lib = None


def build() -> str:
    os.makedirs(os.path.dirname(LIBRARY), exist_ok=True)
    tmp = LIBRARY + ".tmp"
    subprocess.run(GCC_CMD + [SOURCE, "-o", tmp, "-lm"], check=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY) or os.path.getmtime(LIBRARY) < os.path.getmtime(SOURCE):
            build()
        lib = ctypes.CDLL(LIBRARY)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        i64 = ctypes.c_int64
        lib.oracle_scan_f32.restype = None
        lib.oracle_scan_f32.argtypes = [f32p, f32p, f32p, ctypes.c_void_p, ctypes.c_void_p, i64, i64, i64, i64, i64]
        lib.oracle_step_f32.restype = None
        lib.oracle_step_f32.argtypes = [f32p, f32p, f32p, f32p, f32p, ctypes.c_void_p, i64, i64, i64, i64]
        lib.oracle_bruteforce_f64.restype = None
        lib.oracle_bruteforce_f64.argtypes = [f64p, f64p, f64p, i64, i64, i64, i64]
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def scan_f32(lam, V, init=None, t_offset=0):
    """V: float32 [B,H,N,D] (numpy).  Returns (out, final_state) float32."""
    V = np.ascontiguousarray(V, dtype=np.float32)
    lam = np.ascontiguousarray(lam, dtype=np.float32)
    B, H, N, D = V.shape
    out = np.empty_like(V)
    fin = np.empty((B, H, D), np.float32)
    init = None if init is None else np.ascontiguousarray(init, dtype=np.float32)
    load().oracle_scan_f32(V, lam, out, _ptr(init), _ptr(fin), B, H, N, D, int(t_offset))
    return out, fin


def step_f32(lam, state, v, t_pos):
    """One decode step; t_pos int or sequence of B ints.  Returns (out, new_state)."""
    state = np.ascontiguousarray(state, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    lam = np.ascontiguousarray(lam, dtype=np.float32)
    B, H, D = state.shape
    s_out = np.empty_like(state)
    out = np.empty_like(state)
    if isinstance(t_pos, int):
        load().oracle_step_f32(lam, state, v, s_out, out, None, t_pos, B, H, D)
    else:
        tp = np.ascontiguousarray(t_pos, dtype=np.int64)
        load().oracle_step_f32(lam, state, v, s_out, out, _ptr(tp), 0, B, H, D)
    return out, s_out


def bruteforce_f64(lam, V):
    V = np.ascontiguousarray(V, dtype=np.float64)
    lam = np.ascontiguousarray(lam, dtype=np.float64)
    B, H, N, D = V.shape
    out = np.empty_like(V)
    load().oracle_bruteforce_f64(V, lam, out, B, H, N, D)
    return out
