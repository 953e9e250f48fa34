#!/usr/bin/env python3
"""Benchmark of the global-decay scan on one MI355X.

Workload (the metric's configuration): full-sequence decay scan, bf16 V and y,
fp32 arithmetic, B=8 N=4096 H=12 D=64 (25.2 M elements, 100.66 MB of
algorithmic traffic per launch: one read of V, one write of y).  A step is one
launch of the scan over one batch; inputs are resident in HBM and the step
rotates over 8 (V, y) buffer sets (400 MB of V, 400 MB of y), so neither the
inputs nor the outputs fit the 256 MB Infinity Cache between launches.

Prints one JSON line.  Also measured (under "extras"): the box's copy
bandwidth, the decode step (C3: 256 x 12 x 64, launch-latency bound) and the
long-context scan (C4: B=1 N=65536 H=16 D=128 bf16).  The CPU baseline is the
oracle's restatement of the reference's CPU path timed on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extras]
                    [--workload c2|c5_layer|c4]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decay-scan HBM GB/s (% of peak) + tokens/sec, B=8 N=4096 H=12 Dh=64 bf16"
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, vendor peak


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    # 1000 warm-up launches (about 18 ms): after 20 the device had not reached its
    # steady clocks and the same build measured 18.2-18.9 us per C2 step, against
    # 17.9 us after 2000 (four runs on one box).
    p.add_argument("--warmup", type=int, default=1000)
    p.add_argument("--rotate", type=int, default=8, help="(V, y) buffer sets cycled through")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true")
    # The headline line is C2.  The other two time the same protocol (warm-up,
    # rotated sets, HIP-event region) on another shape, for profiling one
    # kernel shape alone; they print no extras and no CPU baseline.
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="c2")
    return p.parse_args()


# name -> (B, H, N, D, description); bf16 V and y.  lam as C2's (one head at 0.9999).
WORKLOADS = {
    "c2": (8, 12, 4096, 64, "full-sequence global-decay scan, bf16 V/y, fp32 accumulate"),
    "c5_layer": (8, 6, 1024, 64, "one layer of the end-to-end model's decay path (C5), bf16 V/y"),
    "c4": (1, 16, 65536, 128, "long-context scan (C4), bf16 V/y"),
}


def c2_lam(H: int, torch):
    g = torch.Generator().manual_seed(1)
    u = 0.5 + (0.9999 - 0.5) * torch.rand(H, generator=g, dtype=torch.float64)
    lam = torch.sigmoid(torch.log(u / (1 - u)).float())
    lam[H - 1] = 0.9999
    return lam


class ScanLauncher:
    """Direct C-ABI launches (no Python tensor plumbing inside the timed loop)."""

    def __init__(self, torch, kilat_amd, lam, sets, code):
        from kilat_amd import _lib
        from kilat_amd.triton_ops import _stream_ptr, _workspace

        self.lib = _lib.load()
        V0 = sets[0][0]
        B, H, N, D = V0.shape
        dev = V0.device
        self.stream = _stream_ptr(dev)
        nbytes = self.lib.kdecay_scan_workspace_bytes(B, H, N, D, code)
        ws = _workspace(dev, self.stream, nbytes)
        self.args = []
        for V, y in sets:
            self.args.append((
                V.data_ptr(), code, _lib.strides4(V.stride()), y.data_ptr(), code, _lib.strides4(y.stride()),
                lam.data_ptr(), None, None, B, H, N, D, 0,
                ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, self.stream,
            ))
        self.fn = self.lib.kdecay_scan_fwd
        self.rc = 0

    def __call__(self, k: int) -> None:
        self.rc |= self.fn(*self.args[k % len(self.args)])


def carved_pairs(torch, dev, shape, ti, to, count: int, seed: int):
    """`count` (V, y) pairs of dtypes (ti, to) carved back to back from one byte
    allocation, V filled with randn (as rotated_sets, for any pair of types)."""
    n = 1
    for d in shape:
        n *= d
    ei, eo = torch.empty(0, dtype=ti).element_size(), torch.empty(0, dtype=to).element_size()
    buf = torch.empty(count * n * (ei + eo), dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    sets, off = [], 0
    for _ in range(count):
        V = buf[off:off + n * ei].view(ti).view(*shape)
        off += n * ei
        y = buf[off:off + n * eo].view(to).view(*shape)
        off += n * eo
        V.copy_(torch.randn(*shape, generator=g, device=dev))
        sets.append((V, y))
    return sets


def rotated_sets(torch, dev, shape, count: int, seed: int = 1):
    """`count` (V, y) bf16 pairs carved from one allocation, V filled with randn.

    One allocation keeps the buffers contiguous in the device address space;
    separate caching-allocator blocks measured about 3% slower for the same
    launches (the scan is HBM-bound, so page placement shows)."""
    n = 1
    for d in shape:
        n *= d
    buf = torch.empty(2 * count * n, dtype=torch.bfloat16, device=dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for k in range(count):
        V = buf[2 * k * n:(2 * k + 1) * n].view(*shape)
        V.copy_(torch.randn(*shape, generator=g, device=dev))
        sets.append((V, buf[(2 * k + 1) * n:(2 * k + 2) * n].view(*shape)))
    return sets


# Wall time each extra measurement keeps launching before its timed region.
# After an idle gap (its buffers being allocated and filled) the device runs a
# memory-bound kernel slower for about 10 ms: back-to-back regions of 100 C2
# training-forward launches in a fresh process measured 18.7, 19.1, 18.4, 17.9,
# 17.4, then 17.0-17.1 us per launch, and a backward timed after only 100
# warm-up launches read 28.6-29.2 us against 26.8-27.2 us once past that ramp
# (one second of copies or matmuls before the allocation did not remove it).
EXTRA_WARM_MS = 30.0


def warm(torch, launch, ms: float, start: int = 0, batch: int = 64) -> int:
    """Launch in batches until `ms` of wall time have passed, then synchronise;
    returns the next launch index."""
    k, t = start, time.perf_counter()
    while True:
        torch.cuda.synchronize()
        if time.perf_counter() - t >= ms * 1e-3:
            return k
        for _ in range(batch):
            launch(k)
            k += 1


def time_region(torch, launch, steps: int, warmup: int, events: bool = True, warm_ms: float = 0.0):
    """(region ms over `steps` launches, per-launch event durations in ms, or
    an empty list without `events`).

    `warmup` launches first, then, with `warm_ms`, more until that much wall
    time has passed (the extras; the headline keeps exactly the --warmup count
    it is given)."""
    for k in range(warmup):
        launch(k)
    if warm_ms > 0:
        warm(torch, launch, warm_ms, warmup)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for k in range(steps):
        launch(k)
    t1.record()
    torch.cuda.synchronize()
    region = t0.elapsed_time(t1)
    if not events:
        return region, []
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for k in range(steps):
        evs[k][0].record()
        launch(k)
        evs[k][1].record()
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) for a, b in evs]
    return region, per


def copy_bandwidth(torch, dev) -> float:
    n = 128 * 1024 * 1024  # 256 MB of bf16 per buffer
    bufs = [(torch.empty(n, dtype=torch.bfloat16, device=dev), torch.empty(n, dtype=torch.bfloat16, device=dev))
            for _ in range(2)]
    for a, b in bufs:
        a.fill_(1.0)

    def launch(k):
        a, b = bufs[k % 2]
        b.copy_(a)

    region, _ = time_region(torch, launch, 20, 4, warm_ms=EXTRA_WARM_MS)
    return 2 * n * 2 * 20 / (region * 1e-3) / 1e9


def bench_decode(torch, kilat_amd, dev, steps=500):
    from kilat_amd import _lib

    S, H, D = 256, 12, 64
    g = torch.Generator(device=dev).manual_seed(2)
    lam = c2_lam(H, torch).to(dev)
    state = torch.randn(S, H, D, generator=g, device=dev)
    v = torch.randn(S, H, D, generator=g, device=dev).to(torch.bfloat16)
    tpos = torch.randint(1, 2049, (S,), generator=g, device=dev, dtype=torch.int32)
    out = torch.empty(S, H, D, device=dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = (lam.data_ptr(), state.data_ptr(), v.data_ptr(), _lib.KDECAY_BF16, state.data_ptr(), out.data_ptr(),
            _lib.KDECAY_F32, tpos.data_ptr(), 0, S, H, D, stream)
    rc = [0]

    def launch(k):
        rc[0] |= lib.kdecay_step(*args)

    region, per = time_region(torch, launch, steps, 20, warm_ms=EXTRA_WARM_MS)
    if rc[0]:
        raise RuntimeError("kdecay_step failed")
    us = region * 1e3 / steps
    # The same steps replayed from a HIP graph: 128 launches captured once, so
    # the host launch cost is gone and the per-step figure is the GPU's own.
    gsteps = 128
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        gargs = list(args)
        gargs[-1] = side.cuda_stream
        with torch.cuda.graph(graph, stream=side):
            for _ in range(gsteps):
                rc[0] |= lib.kdecay_step(*gargs)
    torch.cuda.synchronize()
    warm(torch, lambda k: graph.replay(), EXTRA_WARM_MS, batch=1)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(5):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    if rc[0]:
        raise RuntimeError("kdecay_step failed under capture")
    us_graph = t0.elapsed_time(t1) * 1e3 / (5 * gsteps)
    nbytes = S * H * D * (4 + 2 + 4 + 4)
    return {"config": "C3: 256 seqs x 12 heads x 64, bf16 v_t, fp32 state, per-sequence t_pos",
            "us_per_step": round(us, 3), "us_per_step_graph": round(us_graph, 3),
            "kernel_us_events": round(statistics.median(per) * 1e3, 3),
            "tokens_per_s": round(S / (us * 1e-6), 1), "tokens_per_s_graph": round(S / (us_graph * 1e-6), 1),
            "bytes_per_step": nbytes, "GBps_graph": round(nbytes / (us_graph * 1e-6) / 1e9, 1)}


def bench_decode_layers(torch, kilat_amd, dev, replays=200):
    """One token's decay steps through every layer of the C5 model (12 layers x
    6 heads x 64 channels, bf16 v_t, fp32 state updated in place, positions in
    device memory advanced inside the graph), captured once as a HIP graph and
    replayed once per token, for a decode batch of 8 and of 256 sequences."""
    L, H, D = 12, 6, 64
    res = {"config": "C5 decode: 12 layers x 6 heads x 64 per token, one HIP graph per token"}
    for B in (8, 256):
        g = torch.Generator(device=dev).manual_seed(6)
        lams = [c2_lam(H, torch).to(dev) for _ in range(L)]
        st = [torch.randn(B, H, D, generator=g, device=dev) for _ in range(L)]
        v_in = torch.randn(L, B, H, D, generator=g, device=dev).to(torch.bfloat16)
        outs = torch.empty(L, B, H, D, device=dev)
        tpos = torch.randint(1, 2049, (B,), generator=g, device=dev, dtype=torch.int32)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for l in range(L):
                    kilat_amd.decay_step(lams[l], st[l], v_in[l], tpos, out=outs[l], new_state=st[l])
                tpos.add_(1)
        torch.cuda.synchronize()
        warm(torch, lambda k: graph.replay(), EXTRA_WARM_MS, batch=1)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(replays):
            graph.replay()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / replays
        res[f"B{B}"] = {"us_per_token": round(us, 3), "us_per_layer": round(us / L, 3),
                        "tokens_per_s": round(B / (us * 1e-6), 1),
                        "bytes_per_token": L * B * H * D * (4 + 2 + 4 + 4)}
    return res


def bench_long(torch, kilat_amd, dev, steps=20):
    B, H, N, D = 1, 16, 65536, 128
    u = 0.99 + (0.99999 - 0.99) * torch.rand(H, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    lam = torch.sigmoid(torch.log(u / (1 - u)).float()).to(dev)
    sets = rotated_sets(torch, dev, (B, H, N, D), 2, seed=3)
    from kilat_amd import _lib

    launch = ScanLauncher(torch, kilat_amd, lam, sets, _lib.KDECAY_BF16)
    region, per = time_region(torch, launch, steps, 3, warm_ms=EXTRA_WARM_MS)
    if launch.rc:
        raise RuntimeError("kdecay_scan_fwd failed")
    nbytes = B * H * N * D * 4
    kern = statistics.mean(per)
    gbps = nbytes * steps / (region * 1e-3) / 1e9
    # As for the headline metric: the region average per launch.  The
    # per-launch event pairs add their own overhead and are reported apart.
    return {"config": "C4: B=1 N=65536 H=16 D=128 bf16", "ms_per_step": round(region / steps, 5),
            "GBps": round(gbps, 1), "pct_of_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "event_bracketed_GBps": round(nbytes / (kern * 1e-3) / 1e9, 1),
            "tokens_per_s": round(B * N / (region / steps * 1e-3), 1)}


def measured_traffic(workload: str = "c2"):
    """HBM bytes per launch of the workload's scan from the committed rocprofv3 PMC summary, or None.

    profiles/scan_chunked_bf16_c2_counters.json holds FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch) of the scan at each workload and of a copy kernel of
    known size, which gives the factor each counter is scaled by.
    """
    path = os.path.join(ROOT, "profiles", "scan_chunked_bf16_c2_counters.json")
    key = {"c2": "scan", "c4": "scan_c4", "c5_layer": "scan_c5_layer"}[workload]
    try:
        with open(path) as f:
            m = json.load(f)
        return int(round(m[key]["fetch_kib"] * m["fetch_scale"] * 1024 + m[key]["write_kib"] * m["write_scale"] * 1024))
    except (OSError, KeyError, ValueError):
        return None


def bench_forward_dtypes(torch, dev, steps=100):
    """The C2 shape (B=8 N=4096 H=12) with other I/O types than the headline's
    bf16: fp16, fp32 in and out (D=64: two 128-byte channel groups per head, so
    twice the bytes; D=32: C2's bytes), bf16 in / fp32 out, bf16 with D=128
    (twice the bytes) and fp64 in and out (D=64: four 128-byte channel groups
    per head, four times the bytes).  Algorithmic bytes: V read once, y
    written once.
    4 rotated sets, carved from one allocation as the headline's are (fp16 in
    separate caching-allocator blocks measured 18.2 us against 17.6 us carved,
    the same as bf16 either way)."""
    from kilat_amd import _lib
    from kilat_amd.triton_ops import _stream_ptr, _workspace

    B, H, N = 8, 12, 4096
    lib = _lib.load()
    codes = {torch.float32: _lib.KDECAY_F32, torch.bfloat16: _lib.KDECAY_BF16, torch.float16: _lib.KDECAY_F16,
             torch.float64: _lib.KDECAY_F64}
    lam = c2_lam(H, torch).to(dev)
    stream = _stream_ptr(dev)
    out = {}
    for name, ti, to, D in (("f16", torch.float16, torch.float16, 64), ("f32_d64", torch.float32, torch.float32, 64),
                            ("f32_d32", torch.float32, torch.float32, 32),
                            ("bf16_in_f32_out", torch.bfloat16, torch.float32, 64),
                            ("bf16_d128", torch.bfloat16, torch.bfloat16, 128),
                            ("f64_d64", torch.float64, torch.float64, 64)):
        sets = carved_pairs(torch, dev, (B, H, N, D), ti, to, 4, seed=11)
        nb = lib.kdecay_scan_workspace_bytes(B, H, N, D, codes[ti])
        ws = _workspace(dev, stream, nb)
        args = [(V.data_ptr(), codes[ti], _lib.strides4(V.stride()), y.data_ptr(), codes[to], _lib.strides4(y.stride()),
                 lam.data_ptr(), None, None, B, H, N, D, 0, ws.data_ptr(), ws.numel(), stream) for V, y in sets]
        rc = [0]

        def launch(k, args=args, rc=rc):
            rc[0] |= lib.kdecay_scan_fwd(*args[k % len(args)])

        region, _ = time_region(torch, launch, steps, 200, events=False, warm_ms=EXTRA_WARM_MS)
        if rc[0]:
            raise RuntimeError("scan failed: " + lib.kdecay_last_error_string().decode())
        us = region * 1e3 / steps
        nbytes = B * H * N * D * (sets[0][0].element_size() + sets[0][1].element_size())
        out[name] = {"D": D, "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "pct_of_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 2)}
        del sets, args
    return out


def bench_forward_grids(torch, dev, steps=50):
    """bf16 D=64 N=4096 grids of more than one resident round of 512-row
    chunks, which the library runs as batch slices of whole CU rounds: B=16
    and B=24 at H=12 (two and three launches of 768 chunks) and the larger
    sample configuration's decay heads (H=16 of 64 channels) at B=12 (two
    launches of 768).  Algorithmic bytes: V read once, y written once; 4
    rotated sets carved from one allocation."""
    from kilat_amd import _lib
    from kilat_amd.triton_ops import _stream_ptr, _workspace

    N, D = 4096, 64
    lib = _lib.load()
    code = _lib.KDECAY_BF16
    stream = _stream_ptr(dev)
    out = {}
    for name, B, H in (("B16_H12", 16, 12), ("B24_H12", 24, 12), ("B12_H16", 12, 16)):
        lam = c2_lam(H, torch).to(dev)
        sets = carved_pairs(torch, dev, (B, H, N, D), torch.bfloat16, torch.bfloat16, 4, seed=13)
        ws = _workspace(dev, stream, lib.kdecay_scan_workspace_bytes(B, H, N, D, code))
        args = [(V.data_ptr(), code, _lib.strides4(V.stride()), y.data_ptr(), code, _lib.strides4(y.stride()),
                 lam.data_ptr(), None, None, B, H, N, D, 0, ws.data_ptr(), ws.numel(), stream) for V, y in sets]
        rc = [0]

        def launch(k, args=args, rc=rc):
            rc[0] |= lib.kdecay_scan_fwd(*args[k % len(args)])

        region, _ = time_region(torch, launch, steps, 100, events=False, warm_ms=EXTRA_WARM_MS)
        if rc[0]:
            raise RuntimeError("scan failed: " + lib.kdecay_last_error_string().decode())
        us = region * 1e3 / steps
        nbytes = B * H * N * D * 4
        out[name] = {"B": B, "H": H, "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "pct_of_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 2)}
        del sets, args
    return out


def bench_backward(torch, dev, steps=100, B=8, H=12):
    """C2-shaped training pass (or another batch and head count at N=4096
    D=64): kdecay_scan_fwd_train, then kdecay_scan_bwd (dV, dlam).

    Algorithmic bytes: forward 4 B/element (V in, y out); backward 6 B/element
    (V and gy in, dV out).  4 rotated buffer sets (400 MB of V and gy) keep the
    inputs out of the 256 MB Infinity Cache.
    """
    from kilat_amd import _lib
    from kilat_amd.triton_ops import _stream_ptr, _workspace

    N, D = 4096, 64
    lib = _lib.load()
    code = _lib.KDECAY_BF16
    g = torch.Generator(device=dev).manual_seed(5)
    lam = c2_lam(H, torch).to(dev)
    stream = _stream_ptr(dev)
    nst = lib.kdecay_scan_saved_states_floats(B, H, N, D, code)
    nbytes = max(lib.kdecay_scan_workspace_bytes(B, H, N, D, code), lib.kdecay_scan_bwd_workspace_bytes(B, H, N, D, code))
    ws = _workspace(dev, stream, nbytes)
    sets = []
    nset = 4
    # V, gy, y and dV of every set carved from one allocation, as the headline's
    # sets are (separate caching-allocator blocks measured slower).
    n = B * H * N * D
    buf = torch.empty(4 * nset * n, dtype=torch.bfloat16, device=dev)
    for k in range(nset):
        V, gy, y, dV = (buf[(4 * k + j) * n:(4 * k + j + 1) * n].view(B, H, N, D) for j in range(4))
        V.copy_(torch.randn(B, H, N, D, generator=g, device=dev))
        gy.copy_(torch.randn(B, H, N, D, generator=g, device=dev))
        sets.append((V, gy, y, dV, torch.empty(nst, device=dev), torch.empty(H, device=dev),
                     torch.empty(B, H, D, device=dev)))
    st = _lib.strides4(sets[0][0].stride())
    rc = [0]

    def fwd(k):
        V, gy, y, dV, states, dlam, fin = sets[k % nset]
        rc[0] |= lib.kdecay_scan_fwd_train(V.data_ptr(), code, st, y.data_ptr(), code, st, lam.data_ptr(), None,
                                           fin.data_ptr(), states.data_ptr(), nst, B, H, N, D, 0, ws.data_ptr(),
                                           ws.numel(), stream)

    def bwd(k):
        V, gy, y, dV, states, dlam, fin = sets[k % nset]
        rc[0] |= lib.kdecay_scan_bwd(V.data_ptr(), code, st, gy.data_ptr(), st, dV.data_ptr(), st, lam.data_ptr(),
                                     None, states.data_ptr(), None, dlam.data_ptr(), None, B, H, N, D, 0,
                                     ws.data_ptr(), ws.numel(), stream)

    rf, _ = time_region(torch, fwd, steps, 100, events=False, warm_ms=EXTRA_WARM_MS)
    rb, _ = time_region(torch, bwd, steps, 100, events=False, warm_ms=EXTRA_WARM_MS)
    if rc[0]:
        raise RuntimeError("training scan failed: " + lib.kdecay_last_error_string().decode())
    fus, bus = rf * 1e3 / steps, rb * 1e3 / steps
    config = "C2 shape" if (B, H) == (8, 12) else f"B={B} H={H} N=4096 D=64"
    return {"config": config + ", bf16: forward with saved states, then backward (dV, dlam)",
            "fwd_train_us": round(fus, 3), "fwd_train_GBps": round(4 * n / (fus * 1e-6) / 1e9, 1),
            "bwd_us": round(bus, 3), "bwd_GBps": round(6 * n / (bus * 1e-6) / 1e9, 1),
            "bwd_pct_of_peak": round(100 * 6 * n / (bus * 1e-6) / 1e9 / HBM_PEAK_GBPS, 2)}


def bench_e2e(torch, dev, iters=5):
    """C5: KilatTransformer forward (768 wide, 12 layers, 6 decay + 6 MLA heads, MoE 8 x top-2,
    vocab 50000), random init, bf16 autocast, B=8 N=1024, decay path on the HIP kernel, with
    the reference's glue (two .contiguous() copies around the op) and with layout-fused I/O.

    The model is host-bound (its MoE expert loop synchronises with the host), so its
    forward time hides the decay path; the path itself is timed apart, GPU-bound, by
    decay_path_per_layer()."""
    import kilat_amd
    from tests.e2e_model import E2EConfig, KilatE2E

    torch.manual_seed(4)
    cfg = E2EConfig()
    B, N = 8, 1024
    model = KilatE2E(cfg, kilat_amd.triton_global_decay).to(dev).eval()
    ids = torch.randint(0, cfg.vocab_size, (B, N), device=dev)
    out = {"config": "C5: n_embd=768 n_layer=12 n_head=12 recall_ratio=0.5 MoE 8 x top-2 (+2 shared) "
                     "vocab=50000, bf16 autocast, B=8 N=1024, random init"}
    for fused in (False, True):
        model.set_decay(kilat_amd.triton_global_decay, fused_layout=fused)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            for _ in range(2):
                model(ids)
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(iters):
                model(ids)
            torch.cuda.synchronize()
            sec = (time.perf_counter() - t) / iters
        key = "fused_layout" if fused else "reference_glue"
        out[key] = {"ms_per_forward": round(sec * 1e3, 3), "tokens_per_s": round(B * N / sec, 1)}
    out["decay_path_per_layer"] = decay_path_per_layer(torch, dev)
    out["prefill_with_cache"] = bench_prefill_cache(torch, dev, model, ids)
    return out


def bench_prefill_cache(torch, dev, model, ids, iters=3):
    """C5 prefill with use_cache: the decay state each layer hands to decoding.

    The reference seeds it after the full-sequence op with an N-step loop of
    two torch ops per step (attention.py:383-394); here the scan returns it
    with y from the same launch (return_final_state).  Timed for the whole C5
    model forward with use_cache (both with the layout-fused op), and for one
    layer's seed alone at the C5 shape: the loop, against one scan launch that
    returns y and the state."""
    import kilat_amd
    from tests.e2e_model import KernelDecayCache, ReferenceDecayCache

    B, N = ids.shape
    out = {"config": "C5 model forward with use_cache (B=8 N=1024, bf16 autocast), and one layer's "
                     "decay-state seed at B=8 N=1024 H=6 D=64 bf16"}
    for key, ops in (("reference_seed_loop", ReferenceDecayCache()), ("scan_final_state", KernelDecayCache())):
        model.set_decay(kilat_amd.triton_global_decay, fused_layout=True, cache_ops=ops)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            model(ids, use_cache=True)
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(iters):
                model(ids, use_cache=True)
            torch.cuda.synchronize()
            sec = (time.perf_counter() - t) / iters
        out[key] = {"ms_per_prefill": round(sec * 1e3, 3), "tokens_per_s": round(B * N / sec, 1)}
    model.set_decay(kilat_amd.triton_global_decay, fused_layout=False, cache_ops=ReferenceDecayCache())

    H, D = 6, 64
    g = torch.Generator(device=dev).manual_seed(7)
    V = torch.randn(B, H, N, D, generator=g, device=dev).to(torch.bfloat16)
    lam = c2_lam(H, torch).to(dev)
    layer = {}
    for key, ops, reps in (("reference_seed_loop_us", ReferenceDecayCache(), 3),
                           ("scan_with_final_state_us", KernelDecayCache(), 200)):
        warm(torch, lambda k: ops.prefill(kilat_amd.triton_global_decay, lam, V, torch.float32), EXTRA_WARM_MS,
             batch=1)
        t = time.perf_counter()
        for _ in range(reps):
            ops.prefill(kilat_amd.triton_global_decay, lam, V, torch.float32)
        torch.cuda.synchronize()
        layer[key] = round((time.perf_counter() - t) / reps * 1e6, 2)
    out["per_layer"] = layer
    return out


def decay_path_per_layer(torch, dev, reps=200):
    """One layer's decay path at the C5 shape, GPU-bound (many layers' worth of launches
    back to back, 16 rotated projection buffers): from the v_proj_global output (B,N,H*D)
    to the (B,N,H*D) input of the concatenation.  'reference_glue' is attention.py:368-374
    (.view/.transpose/.contiguous(), the op, .transpose/.reshape: two copies and the scan),
    'fused_layout' hands the op the strided view and takes its output back as a view (the
    scan alone).  Also the scan alone on contiguous V, through the C ABI."""
    import kilat_amd
    from kilat_amd import _lib

    B, N, H, D = 8, 1024, 6, 64
    lam = c2_lam(H, torch).to(dev)
    flats = [torch.randn(B, N, H * D, device=dev).to(torch.bfloat16) for _ in range(16)]

    def glue(k):
        V = flats[k % 16].view(B, N, H, D).transpose(1, 2).contiguous()
        return kilat_amd.triton_global_decay(lam, V).transpose(1, 2).reshape(B, N, H * D)

    def fused(k):
        V = flats[k % 16].view(B, N, H, D).transpose(1, 2)
        return kilat_amd.triton_global_decay(lam, V).transpose(1, 2).reshape(B, N, H * D)

    lib = _lib.load()
    conts = [f.view(B, N, H, D).transpose(1, 2).contiguous() for f in flats]
    ys = [torch.empty_like(c) for c in conts]
    from kilat_amd.triton_ops import _stream_ptr, _workspace

    stream = _stream_ptr(dev)
    ws = _workspace(dev, stream, lib.kdecay_scan_workspace_bytes(B, H, N, D, _lib.KDECAY_BF16))
    args = [(c.data_ptr(), _lib.KDECAY_BF16, _lib.strides4(c.stride()), y.data_ptr(), _lib.KDECAY_BF16,
             _lib.strides4(y.stride()), lam.data_ptr(), None, None, B, H, N, D, 0, ws.data_ptr(), ws.numel(), stream)
            for c, y in zip(conts, ys)]

    rc = [0]

    def scan_only(k):
        rc[0] |= lib.kdecay_scan_fwd(*args[k % 16])

    res = {"config": "one layer at C5: B=8 N=1024 H=6 D=64 bf16, GPU-bound back-to-back, 16 rotated buffers"}
    for name, fn in (("reference_glue", glue), ("fused_layout", fused), ("scan_only_c_abi", scan_only)):
        # the graph keeps the host out of the measurement: reps layers captured once
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for k in range(4):
                fn(k)  # eager warm-up on the capture stream (sizes its workspace)
            if name == "scan_only_c_abi":  # its launches go to the capture stream from here on
                args[:] = [a[:-1] + (side.cuda_stream,) for a in args]
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for k in range(reps):
                    fn(k)
        # the eager warm-up launches and the captured ones were all accepted
        if rc[0]:
            raise RuntimeError("kdecay_scan_fwd failed: " + lib.kdecay_last_error_string().decode())
        torch.cuda.synchronize()
        warm(torch, lambda k: g.replay(), EXTRA_WARM_MS, batch=1)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(3):
            g.replay()
        t1.record()
        torch.cuda.synchronize()
        res[name + "_us"] = round(t0.elapsed_time(t1) * 1e3 / (3 * reps), 3)
        del g
    return res


def cpu_baseline(torch, B, H, N, D):
    """The oracle's torch restatement of the reference CPU path on the host cores."""
    from oracle import decay_oracle as O

    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        cores = min(cores, int(env))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(1)
    V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).float()
    lam = c2_lam(H, torch)
    O.global_decay(lam, V[:, :, :64])  # warm-up
    times = []
    for _ in range(3):
        t = time.perf_counter()
        O.global_decay(lam, V)
        times.append(time.perf_counter() - t)
    sec = statistics.median(times)
    nbytes = B * H * N * D * 4  # same algorithmic bytes as the GPU line (bf16 in + out)
    return {"value": round(nbytes / sec / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full workload B={B} N={N} H={H} D={D} (bf16-rounded V as fp32), median of 3 runs after a warm-up",
            "seconds": round(sec, 4), "tokens_per_s": round(B * N / sec, 1)}


def cpu_extras(torch):
    """The same CPU restatement on BASELINE's other configurations (host cores,
    fp32 arithmetic): C1 (the reference's CPU-op case), C3 (the incremental
    step with the batch-shared t_pos of attention.py:344-360) and C4 (one
    timed run of the 65,536-step loop)."""
    from oracle import decay_oracle as O

    out = {}
    g = torch.Generator().manual_seed(0)
    V = torch.randn(2, 6, 1024, 64, generator=g)
    u = 0.90 + (0.999 - 0.90) * torch.rand(6, generator=g, dtype=torch.float64)
    lam = torch.sigmoid(torch.log(u / (1 - u)).float())
    O.global_decay(lam, V[:, :, :32])
    times = []
    for _ in range(3):
        t = time.perf_counter()
        O.global_decay(lam, V)
        times.append(time.perf_counter() - t)
    sec = statistics.median(times)
    out["C1"] = {"config": "B=2 N=1024 H=6 D=64 fp32", "seconds": round(sec, 4),
                 "tokens_per_s": round(2 * 1024 / sec, 1), "GBps": round(V.numel() * 8 / sec / 1e9, 4)}

    g = torch.Generator().manual_seed(2)
    S, H, D, steps = 256, 12, 64, 128
    lam = c2_lam(H, torch)
    state0 = torch.randn(S, H, D, generator=g)
    vs = torch.randn(steps, S, H, D, generator=g).to(torch.bfloat16)
    O.step(lam, state0, vs[0], 100)
    state = state0
    t = time.perf_counter()
    for k in range(steps):
        _, state = O.step(lam, state, vs[k], 1000 + k)
    sec = time.perf_counter() - t
    # The same steps on the GPU from the same start, checked against the
    # restatement: the new state must be bit-identical after every step.
    import kilat_amd

    dev = torch.device("cuda", 0)
    lam_d, st_gpu, st_cpu, same = lam.to(dev), state0.to(dev), state0, 0
    for k in range(steps):
        _, st_cpu = O.step(lam, st_cpu, vs[k], 1000 + k)
        _, st_gpu = kilat_amd.decay_step(lam_d, st_gpu, vs[k].to(dev), 1000 + k)
        same += int(torch.equal(st_gpu.cpu(), st_cpu))
    out["C3_step"] = {"config": "256 x 12 x 64, bf16 v_t, fp32 state, batch-shared t_pos, 128 steps",
                      "us_per_step": round(sec / steps * 1e6, 2), "tokens_per_s": round(S * steps / sec, 1),
                      "gpu_state_bitwise_steps": f"{same}/{steps}"}

    g = torch.Generator().manual_seed(3)
    V = torch.randn(1, 16, 65536, 128, generator=g).to(torch.bfloat16).float()
    u = 0.99 + (0.99999 - 0.99) * torch.rand(16, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    lam = torch.sigmoid(torch.log(u / (1 - u)).float())
    O.global_decay(lam, V[:, :, :64])
    t = time.perf_counter()
    O.global_decay(lam, V)
    sec = time.perf_counter() - t
    out["C4"] = {"config": "B=1 N=65536 H=16 D=128 (bf16-rounded V as fp32), one run", "seconds": round(sec, 3),
                 "tokens_per_s": round(65536 / sec, 1), "GBps": round(V.numel() * 4 / sec / 1e9, 4)}
    return out


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the decay scan shards over (b, h) streams with no communication)",
              file=sys.stderr, flush=True)
        return 2
    import torch

    import kilat_amd
    from kilat_amd import _lib

    dev = torch.device("cuda", 0)
    B, H, N, D, workload = WORKLOADS[args.workload]
    headline = args.workload == "c2"
    log(f"allocating {args.rotate} x (V, y) bf16 {B}x{H}x{N}x{D}")
    sets = rotated_sets(torch, dev, (B, H, N, D), args.rotate)
    lam = c2_lam(H, torch).to(dev)
    launch = ScanLauncher(torch, kilat_amd, lam, sets, _lib.KDECAY_BF16)
    log(f"timing {args.steps} steps after {args.warmup} warm-up")
    # No per-launch events here: they would add launches with gaps to the
    # kernel trace that profiles/ summarises.
    region, _ = time_region(torch, launch, args.steps, args.warmup, events=False)
    if launch.rc:
        raise RuntimeError("kdecay_scan_fwd failed: " + _lib.load().kdecay_last_error_string().decode())
    if kilat_amd.workspace_error(sets[0][0]):
        raise RuntimeError("scan workspace reports a look-back fault")

    nbytes = B * H * N * D * (2 + 2)
    ms_step = region / args.steps
    value = nbytes / (ms_step * 1e-3) / 1e9
    # Average launch duration of the scan kernel: the HIP-event region on the
    # launch stream over back-to-back launches, divided by the launch count
    # (events around every single launch would add their own gaps).
    achieved = value
    log(f"region {ms_step * 1e3:.2f} us/step")

    metric = METRIC if headline else (f"decay-scan HBM GB/s (% of peak) + tokens/sec, B={B} N={N} H={H} Dh={D} bf16 "
                                      f"({args.workload})")
    result = {
        "metric": metric,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload,
                   "B": B, "N": N, "H": H, "D": D, "io_dtype": "bf16", "rotated_buffer_sets": args.rotate,
                   "parallelism": "single GPU"},
        "tokens_per_s": round(B * N / (ms_step * 1e-3), 1),
        "pct_of_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(args.workload),
                     "kernel_us": round(ms_step * 1e3, 3), "algorithmic_bytes": nbytes},
    }
    extras = {}
    if headline and not args.no_extras:
        # The training pass first, while the headline's sets are still held, so
        # that its buffers are memory the process has not used before, as the
        # headline's are, whatever the other extras allocate and release.
        # Placed after the other extras its figure followed their allocation
        # history (same box, one process each: alone 26.92 us; after the
        # forward-dtypes extra 27.09-27.20 us; after it with the caching
        # allocator emptied, as the extras then ran, 28.15-28.20 us).
        log("training forward + backward (C2 shape)")
        extras["backward"] = bench_backward(torch, dev)
        log("copy bandwidth")
        extras["copy_GBps"] = round(copy_bandwidth(torch, dev), 1)
        del sets, launch
        torch.cuda.empty_cache()
        log("decode step C3")
        extras["decode"] = bench_decode(torch, kilat_amd, dev)
        log("decode token through 12 layers (C5 shape), graph-replayed")
        extras["decode_layers"] = bench_decode_layers(torch, kilat_amd, dev)
        log("long context C4")
        extras["long_context"] = bench_long(torch, kilat_amd, dev)
        torch.cuda.empty_cache()
        log("forward with other I/O types (C2 shape)")
        extras["forward_dtypes"] = bench_forward_dtypes(torch, dev)
        torch.cuda.empty_cache()
        log("forward, grids of more than one round (bf16 D=64 N=4096)")
        extras["forward_grids"] = bench_forward_grids(torch, dev)
        torch.cuda.empty_cache()
        # Backward grids of exactly two resident rounds, which the library runs
        # as two batch slices: B=16 H=12, and the larger sample configuration's
        # decay heads (H=16 of 64 channels) at B=12.
        log("training pass, backward grids of two rounds (bf16 D=64 N=4096)")
        extras["backward_grids"] = {}
        for B2, H2 in ((16, 12), (12, 16)):
            extras["backward_grids"][f"B{B2}_H{H2}"] = bench_backward(torch, dev, steps=50, B=B2, H=H2)
            torch.cuda.empty_cache()
        log("end-to-end model forward (C5)")
        extras["e2e"] = bench_e2e(torch, dev)
    result["extras"] = extras
    if headline and not args.no_cpu_baseline:
        log("CPU baseline (oracle restatement of the reference CPU path)")
        result["cpu_baseline"] = cpu_baseline(torch, B, H, N, D)
        if not args.no_extras:
            log("CPU restatement on C1, C3 and C4")
            result["cpu_baseline"]["extras"] = cpu_extras(torch)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
