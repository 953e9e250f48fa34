"""The ctypes stub the integration guide shows a Kilat maintainer, kept here
verbatim so that tests can run it (tests/test_gpu_scan.py) and check that the
guide still holds this exact text (tests/test_abi.py)."""
from __future__ import annotations

STUB_SOURCE = """\
import ctypes, torch
_kd = ctypes.CDLL("/path/to/libkdecay.so")
_P, _I, _I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
_kd.kdecay_scan_fwd.argtypes = [_P, _I, _P, _P, _I, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                _P, ctypes.c_size_t, _P]
_kd.kdecay_scan_workspace_bytes.restype = ctypes.c_size_t
_kd.kdecay_scan_workspace_bytes.argtypes = [_I64, _I64, _I64, _I64, _I]
_kd.kdecay_last_error_string.restype = ctypes.c_char_p
_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.float64: 3}
_WS = {}    # one zeroed workspace per (device, stream)
_KEEP = []  # replaced workspaces: a captured graph may still use one, so none is ever freed

def _hip_global_decay(lam_scores, V):          # V: [B,H,N,D] on a HIP device, d-stride 1
    B, H, N, D = V.shape
    out = torch.empty_like(V)
    lam = lam_scores.reshape(H).float().contiguous()
    stream = torch.cuda.current_stream(V.device).cuda_stream
    nbytes = _kd.kdecay_scan_workspace_bytes(B, H, N, D, _CODE[V.dtype])
    ws = _WS.get((V.device.index, stream))
    if nbytes and (ws is None or ws.numel() < nbytes):
        _KEEP.append(ws)
        ws = _WS[(V.device.index, stream)] = torch.zeros(nbytes, dtype=torch.uint8, device=V.device)
    st = lambda t: (ctypes.c_int64 * 4)(*t.stride())
    rc = _kd.kdecay_scan_fwd(V.data_ptr(), _CODE[V.dtype], st(V), out.data_ptr(), _CODE[V.dtype], st(out),
                             lam.data_ptr(), None, None, B, H, N, D, 0,
                             ws.data_ptr() if nbytes else None, nbytes, stream)
    if rc:
        raise RuntimeError(_kd.kdecay_last_error_string().decode())
    return out
"""


def load(library_path: str):
    """Execute the stub against `library_path`; returns its _hip_global_decay."""
    ns: dict = {}
    exec(STUB_SOURCE.replace("/path/to/libkdecay.so", library_path), ns)
    return ns["_hip_global_decay"]
