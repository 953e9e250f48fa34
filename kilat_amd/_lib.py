"""ctypes binding of libkdecay.so (declarations: include/kdecay.h).

torch is imported before the library is opened.  torch ships its own HIP
runtime whose SONAME (libamdhip64.so.7) is the one libkdecay.so needs, so the
dynamic linker binds the library to torch's already-loaded runtime: one HIP
runtime per process, and torch's streams and device pointers are valid here.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must load torch's HIP runtime first, see above)

# Built in-tree by kilat_amd/_build.py.
LIBRARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkdecay.so")

KDECAY_F32 = 0
KDECAY_BF16 = 1
KDECAY_F16 = 2
KDECAY_F64 = 3  # the three forward scans only

KDECAY_EINVAL = -1
KDECAY_EDTYPE = -2
KDECAY_ESHAPE = -3
KDECAY_ELAYOUT = -4
KDECAY_EWORKSPACE = -5

KDECAY_NOALLOC_WORKSPACE_BYTES = 8 << 20  # include/kdecay.h

# Every symbol include/kdecay.h declares.
EXPORTS = (
    "kdecay_scan_fwd",
    "kdecay_scan_workspace_bytes",
    "kdecay_scan_fwd_noalloc",
    "kdecay_scan_fwd_train",
    "kdecay_scan_saved_states_floats",
    "kdecay_scan_bwd",
    "kdecay_scan_bwd_workspace_bytes",
    "kdecay_scan_fwd_sequential",
    "kdecay_step",
    "kdecay_version",
    "kdecay_last_error_string",
    "kdecay_debug_set_spin_limit",
    "kdecay_debug_fastdiv",
)

_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p
_c_i64p = ctypes.POINTER(ctypes.c_int64)

_lib = None


def load() -> ctypes.CDLL:
    """Open libkdecay.so once.  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise RuntimeError(
            f"kilat_amd: {LIBRARY} is missing; build it with `python -m kilat_amd._build` "
            "(there is no CPU fallback)"
        )
    lib = ctypes.CDLL(LIBRARY)
    lib.kdecay_scan_fwd.restype = ctypes.c_int
    lib.kdecay_scan_fwd.argtypes = [
        _c_ptr, ctypes.c_int, _c_i64p,      # V, v_dtype, v_strides
        _c_ptr, ctypes.c_int, _c_i64p,      # out, out_dtype, out_strides
        _c_ptr, _c_ptr, _c_ptr,             # lam, init_state, final_state
        _c_i64, _c_i64, _c_i64, _c_i64,     # B, H, N, D
        _c_i64,                             # t_offset
        _c_ptr, ctypes.c_size_t,            # workspace, workspace_bytes
        _c_ptr,                             # stream
    ]
    lib.kdecay_scan_workspace_bytes.restype = ctypes.c_size_t
    lib.kdecay_scan_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int]
    lib.kdecay_scan_fwd_noalloc.restype = ctypes.c_int
    lib.kdecay_scan_fwd_noalloc.argtypes = [
        _c_ptr, ctypes.c_int, _c_i64p,      # V, v_dtype, v_strides
        _c_ptr, ctypes.c_int, _c_i64p,      # out, out_dtype, out_strides
        _c_ptr, _c_ptr, _c_ptr,             # lam, init_state, final_state
        _c_i64, _c_i64, _c_i64, _c_i64,     # B, H, N, D
        _c_i64,                             # t_offset
        _c_ptr,                             # stream
    ]
    lib.kdecay_scan_fwd_train.restype = ctypes.c_int
    lib.kdecay_scan_fwd_train.argtypes = [
        _c_ptr, ctypes.c_int, _c_i64p,      # V, v_dtype, v_strides
        _c_ptr, ctypes.c_int, _c_i64p,      # out, out_dtype, out_strides
        _c_ptr, _c_ptr, _c_ptr,             # lam, init_state, final_state
        _c_ptr, ctypes.c_size_t,            # states, states_floats
        _c_i64, _c_i64, _c_i64, _c_i64,     # B, H, N, D
        _c_i64,                             # t_offset
        _c_ptr, ctypes.c_size_t,            # workspace, workspace_bytes
        _c_ptr,                             # stream
    ]
    lib.kdecay_scan_saved_states_floats.restype = ctypes.c_size_t
    lib.kdecay_scan_saved_states_floats.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int]
    lib.kdecay_scan_bwd.restype = ctypes.c_int
    lib.kdecay_scan_bwd.argtypes = [
        _c_ptr, ctypes.c_int, _c_i64p,      # V, v_dtype, v_strides
        _c_ptr, _c_i64p,                    # gy, gy_strides
        _c_ptr, _c_i64p,                    # dV, dv_strides
        _c_ptr, _c_ptr, _c_ptr, _c_ptr,     # lam, init_state, states, g_final
        _c_ptr, _c_ptr,                     # dlam, d_init
        _c_i64, _c_i64, _c_i64, _c_i64,     # B, H, N, D
        _c_i64,                             # t_offset
        _c_ptr, ctypes.c_size_t,            # workspace, workspace_bytes
        _c_ptr,                             # stream
    ]
    lib.kdecay_scan_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.kdecay_scan_bwd_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int]
    lib.kdecay_scan_fwd_sequential.restype = ctypes.c_int
    lib.kdecay_scan_fwd_sequential.argtypes = [
        _c_ptr, ctypes.c_int, _c_i64p,
        _c_ptr, ctypes.c_int, _c_i64p,
        _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64,
        _c_i64,
        _c_ptr,
    ]
    lib.kdecay_step.restype = ctypes.c_int
    lib.kdecay_step.argtypes = [
        _c_ptr, _c_ptr, _c_ptr, ctypes.c_int,   # lam, state_in, v_t, v_dtype
        _c_ptr, _c_ptr, ctypes.c_int,           # state_out, out, out_dtype
        _c_ptr, _c_i64,                         # t_pos, t_pos_scalar
        _c_i64, _c_i64, _c_i64,                 # B, H, D
        _c_ptr,                                 # stream
    ]
    lib.kdecay_version.restype = ctypes.c_char_p
    lib.kdecay_version.argtypes = []
    lib.kdecay_last_error_string.restype = ctypes.c_char_p
    lib.kdecay_last_error_string.argtypes = []
    lib.kdecay_debug_set_spin_limit.restype = ctypes.c_int
    lib.kdecay_debug_set_spin_limit.argtypes = [ctypes.c_int]
    lib.kdecay_debug_fastdiv.restype = ctypes.c_uint32
    lib.kdecay_debug_fastdiv.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]
    _lib = lib
    return lib


_strides_cache: dict = {}


def strides4(strides) -> ctypes.Array:
    """int64[4] strides for the C ABI, cached per stride tuple (the library
    reads them during the call only, so one array can serve every call)."""
    key = tuple(strides)
    arr = _strides_cache.get(key)
    if arr is None:
        if len(_strides_cache) > 1024:
            _strides_cache.clear()
        arr = _strides_cache[key] = (ctypes.c_int64 * 4)(*[int(s) for s in key])
    return arr


def check(rc: int, what: str) -> None:
    """Raise RuntimeError for a non-zero return code, with the library's message."""
    if rc != 0:
        msg = load().kdecay_last_error_string().decode(errors="replace")
        raise RuntimeError(f"kilat_amd: {what} failed (code {rc}): {msg}")
