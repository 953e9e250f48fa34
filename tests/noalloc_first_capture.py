"""Child process of tests/test_zz_no_alloc.py: the first kdecay_scan_fwd_noalloc
call of a process, made under HIP stream capture.

Nothing else in this process has used the library's device array before the
capture, so the captured scan runs on the array as the code object loader
left it (zero-filled).  The graph is replayed four times, with an eager call
of another shape between replays (which shares the array), and every replay
must give the bits of kdecay_scan_fwd with a workspace of its own.  Prints
"noalloc-first-capture ok" and exits 0, or raises.

Run as a separate process (python tests/noalloc_first_capture.py), never
imported by the test suite.
"""
from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def main() -> int:
    import torch

    from kilat_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(62)
    u = 0.5 + (0.9999 - 0.5) * torch.rand(6, generator=g, dtype=torch.float64)
    lam = torch.sigmoid(torch.log(u / (1 - u)).float()).to(dev)
    B, H, N, D = 8, 6, 3000, 64
    V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev)
    W = torch.randn(2, 6, 5000, 64, generator=g).to(torch.bfloat16).to(dev)
    st, sw = _lib.strides4(V.stride()), _lib.strides4(W.stride())
    bf = _lib.KDECAY_BF16
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    y = torch.empty_like(V)
    fin = torch.empty(B, H, D, device=dev)
    with torch.cuda.stream(side):
        graph = torch.cuda.CUDAGraph()
        print("capturing the first noalloc call of the process", flush=True)
        with torch.cuda.graph(graph, stream=side):
            rc = lib.kdecay_scan_fwd_noalloc(V.data_ptr(), bf, st, y.data_ptr(), bf, st, lam.data_ptr(), None,
                                             fin.data_ptr(), B, H, N, D, 0, side.cuda_stream)
        _lib.check(rc, "noalloc under capture")
    torch.cuda.synchronize()

    def with_workspace(X, sx, out, f):
        b, h, n, d = X.shape
        nb = lib.kdecay_scan_workspace_bytes(b, h, n, d, bf)
        ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
        _lib.check(lib.kdecay_scan_fwd(X.data_ptr(), bf, sx, out.data_ptr(), bf, sx, lam.data_ptr(), None,
                                       f.data_ptr() if f is not None else None, b, h, n, d, 0, ws.data_ptr(),
                                       ws.numel(), torch.cuda.current_stream(dev).cuda_stream), "workspace")
        torch.cuda.synchronize()

    y_ref, f_ref, w_ref = torch.empty_like(V), torch.empty_like(fin), torch.empty_like(W)
    with_workspace(V, st, y_ref, f_ref)
    with_workspace(W, sw, w_ref, None)
    for r in range(4):
        print(f"replay {r}", flush=True)
        y.zero_()
        fin.zero_()
        w = torch.empty_like(W)
        with torch.cuda.stream(side):
            graph.replay()
            _lib.check(lib.kdecay_scan_fwd_noalloc(W.data_ptr(), bf, sw, w.data_ptr(), bf, sw, lam.data_ptr(), None,
                                                   None, 2, 6, 5000, 64, 0, side.cuda_stream), "noalloc eager")
        torch.cuda.synchronize()
        if not (torch.equal(y, y_ref) and torch.equal(fin, f_ref)):
            raise SystemExit(f"replay {r}: captured first call differs from kdecay_scan_fwd")
        if not torch.equal(w, w_ref):
            raise SystemExit(f"replay {r}: eager call between replays differs from kdecay_scan_fwd")
        if not bool(torch.isfinite(y.float()).all()):
            raise SystemExit(f"replay {r}: non-finite output")
    print("noalloc-first-capture ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
