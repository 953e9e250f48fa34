"""kdecay_scan_fwd_noalloc, the entry point that allocates nothing (its
look-back workspace is the library's fixed per-GPU device array), against
kdecay_scan_fwd with a workspace of its own: the same kernels, so the outputs
and final states must be the same bits.  Called through the C ABI (ctypes),
several calls in a row on one GPU, each smaller than the one before, and
replayed from a HIP graph."""
from __future__ import annotations

import pytest
import torch

from kilat_amd import _lib
from oracle import decay_oracle as O
from tests.decay_cases import lam_uniform

pytestmark = pytest.mark.gpu

CODE = {torch.float32: _lib.KDECAY_F32, torch.bfloat16: _lib.KDECAY_BF16, torch.float16: _lib.KDECAY_F16,
        torch.float64: _lib.KDECAY_F64}


def _both(lib, lam, V, init, t_offset, stream):
    """(y, final) from kdecay_scan_fwd with its own zeroed workspace, then from
    kdecay_scan_fwd_noalloc; both enqueued on `stream`."""
    B, H, N, D = V.shape
    code = CODE[V.dtype]
    st = _lib.strides4(V.stride())
    res = []
    for noalloc in (False, True):
        y = torch.empty_like(V)
        fin = torch.empty(B, H, D, device=V.device)
        init_p = init.data_ptr() if init is not None else None
        if noalloc:
            rc = lib.kdecay_scan_fwd_noalloc(V.data_ptr(), code, st, y.data_ptr(), code, st, lam.data_ptr(), init_p,
                                             fin.data_ptr(), B, H, N, D, t_offset, stream)
        else:
            nb = lib.kdecay_scan_workspace_bytes(B, H, N, D, code)
            ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=V.device)
            rc = lib.kdecay_scan_fwd(V.data_ptr(), code, st, y.data_ptr(), code, st, lam.data_ptr(), init_p,
                                     fin.data_ptr(), B, H, N, D, t_offset, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "noalloc" if noalloc else "workspace")
        res.append((y, fin))
    return res


def test_noalloc_matches_workspace_entry_point(hip_device, kdecay_lib):
    lib = kdecay_lib
    stream = torch.cuda.current_stream(hip_device).cuda_stream
    g = torch.Generator().manual_seed(60)
    # each call smaller than the previous one: the array keeps the larger
    # call's words and its epoch, which the next call must not take for its own
    cases = [(16, 12, 4096, 64, torch.bfloat16, True),  # two batch slices on the array, one after the other
             (8, 12, 4096, 64, torch.bfloat16, False), (2, 3, 1500, 64, torch.bfloat16, True),
             (1, 4, 3000, 128, torch.float32, False), (1, 6, 2048, 64, torch.float64, True),
             (1, 2, 700, 32, torch.float16, True),
             (1, 1, 100, 64, torch.bfloat16, False)]
    for k, (B, H, N, D, dt, carry) in enumerate(cases):
        print(f"  noalloc call {k}: B={B} H={H} N={N} D={D} {dt} carry={carry}", flush=True)
        lam = lam_uniform(H, 0.5, 0.9999, g).to(hip_device)
        V = torch.randn(B, H, N, D, generator=g).to(dt).to(hip_device)
        init = torch.randn(B, H, D, generator=g).to(hip_device) if carry else None
        (y0, f0), (y1, f1) = _both(lib, lam, V, init, 17 if carry else 0, stream)
        torch.cuda.synchronize()
        assert torch.equal(y1, y0), k
        assert torch.equal(f1, f0), k
        assert bool(torch.isfinite(y1.float()).all()), k
        if N <= 1500:  # the small ones against the oracle too
            ref, sref = O.scan(lam.cpu(), V.cpu(), None if init is None else init.cpu(), 17 if carry else 0)
            tol = 1e-5 if dt == torch.float32 else 2e-2
            assert float((y1.cpu().double() - ref.double()).abs().max()) <= tol * max(1.0, float(ref.abs().max())), k


def test_noalloc_replays_from_a_graph(hip_device, kdecay_lib):
    """Captured once and replayed, with eager calls of another shape between
    the replays (they share the device array); every replay equals the
    workspace entry point's result."""
    lib = kdecay_lib
    g = torch.Generator().manual_seed(61)
    lam = lam_uniform(6, 0.5, 0.9999, g).to(hip_device)
    V = torch.randn(8, 6, 1024, 64, generator=g).to(torch.bfloat16).to(hip_device)
    W = torch.randn(2, 6, 5000, 64, generator=g).to(torch.bfloat16).to(hip_device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    st = _lib.strides4(V.stride())
    with torch.cuda.stream(side):
        (y_ref, f_ref), _ = _both(lib, lam, V, None, 0, side.cuda_stream)
        (w_ref, _), _ = _both(lib, lam, W, None, 0, side.cuda_stream)
        y = torch.empty_like(V)
        fin = torch.empty(8, 6, 64, device=hip_device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            rc = lib.kdecay_scan_fwd_noalloc(V.data_ptr(), _lib.KDECAY_BF16, st, y.data_ptr(), _lib.KDECAY_BF16, st,
                                             lam.data_ptr(), None, fin.data_ptr(), 8, 6, 1024, 64, 0,
                                             side.cuda_stream)
        _lib.check(rc, "noalloc under capture")
    torch.cuda.synchronize()
    sw = _lib.strides4(W.stride())
    for r in range(4):
        print(f"  noalloc graph replay {r}", flush=True)
        y.zero_()
        fin.zero_()
        with torch.cuda.stream(side):
            graph.replay()
            w = torch.empty_like(W)
            _lib.check(lib.kdecay_scan_fwd_noalloc(W.data_ptr(), _lib.KDECAY_BF16, sw, w.data_ptr(), _lib.KDECAY_BF16,
                                                   sw, lam.data_ptr(), None, None, 2, 6, 5000, 64, 0,
                                                   side.cuda_stream), "noalloc eager")
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref) and torch.equal(fin, f_ref), r
        assert torch.equal(w, w_ref), r


def test_noalloc_first_call_of_a_process_under_capture(hip_device, kdecay_lib):
    """The first no-alloc call of a process made under stream capture: the
    library records no set-up work into the graph (the device array is
    zero-filled by the code object loader, and the library never clears it),
    so the captured scan alone runs on every replay.  Run in a fresh child
    process (a subprocess, so this process's earlier calls do not count)."""
    import os
    import subprocess
    import sys

    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_first_capture.py")
    print("  child process: first noalloc call under capture", flush=True)
    proc = subprocess.run([sys.executable, "-u", script], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=100)
    print(proc.stdout[-2000:], flush=True)
    assert proc.returncode == 0, f"child exited {proc.returncode}"
    assert "noalloc-first-capture ok" in proc.stdout
