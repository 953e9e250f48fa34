"""GPU parity of the full-sequence scan (kdecay_scan_fwd via kilat_amd) against
the CPU oracle, which restates /root/reference/src/kilat/arc/triton_ops.py:232-247.

Tolerances (from the build's target):
  fp32 V:       rel_err <= 1e-5, rel_err = max over (b,h) of max|y - ref| / max|ref|
  bf16/fp16 V:  max|y - ref| <= 2e-2, fp32 accumulation (ref computed from the
                same rounded inputs, output rounded once like the reference)
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import kilat_amd
from kilat_amd import _lib
from oracle import c_oracle as C
from oracle import decay_oracle as O
from tests.decay_cases import (assert_rounded_once, c1_inputs, c2_inputs, c4_inputs, elementwise_rel, lam_uniform,
                               max_abs, rel_err)
from tests.decay_cases import WORKSPACE_HEADER_BYTES as HDR

pytestmark = pytest.mark.gpu

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def chunk_rows(dtype, D, rows_per_lane=16):
    """Rows per chunk of the library's scan: 256 lanes x 16 rows x 16 bytes of one
    channel group of at most 128 bytes (8 rows per lane when the 16-row grid has
    at most 416 chunks, 640 at 2 chunks per stream, 160 at 1)."""
    es = torch.empty((), dtype=dtype).element_size()
    dg = min(D, 128 // es)
    return 4 * (64 // (dg // (16 // es))) * rows_per_lane


def gpu_scan(lam, V, dev, **kw):
    print(f"  scan V{tuple(V.shape)} {V.dtype} {kw}", flush=True)
    res = kilat_amd.global_decay_scan(lam.to(dev), V.to(dev), **kw)
    torch.cuda.synchronize()
    return res


def assert_parity(y, ref, dtype, what=""):
    """fp32: rel_err <= 1e-5.  bf16/fp16: max-abs <= 2e-2 (the target's bound),
    and per (b,h) stream max|y-ref| / max|ref| <= 2e-2 as well, a few ulps of
    the stream's own scale, so that a stream of small values (a head with lam
    near 1 late in the sequence) cannot hide a dropped or wrong carry under
    the absolute bound."""
    if dtype == torch.float32:
        e = rel_err(y, ref)
        assert e <= 1e-5, f"{what}: rel_err {e:.3e} > 1e-5"
    else:
        e = max_abs(y, ref)
        assert e <= 2e-2, f"{what}: max_abs {e:.3e} > 2e-2"
        r = rel_err(y, ref)
        assert r <= 2e-2, f"{what}: per-stream relative error {r:.3e} > 2e-2"


@pytest.mark.parametrize("dname", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
def test_scan_shapes(hip_device, kdecay_lib, dname, D):
    """Small grids (B=2, H=3): the 8-rows-per-lane kernels."""
    dtype = DTYPES[dname]
    L = chunk_rows(dtype, D, 8)
    g = torch.Generator().manual_seed(100 + D)
    lam = lam_uniform(3, 0.5, 0.9999, g)
    for N in sorted({1, 37, L - 1, L, L + 1, 2 * L, 3 * L + 5, 6 * L + 1}):
        V = torch.randn(2, 3, N, D, generator=g).to(dtype)
        y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
        ref, sref = O.scan(lam, V)
        assert y.dtype == dtype and y.shape == V.shape
        assert_parity(y, ref, dtype, f"N={N}")
        assert rel_err(fin, sref) <= 1e-5, f"final state N={N}"


@pytest.mark.parametrize("dname", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
def test_scan_shapes_large_grid(hip_device, kdecay_lib, dname, D):
    """Grids of more than 640 chunks at 16 rows per lane, 2 per stream: the
    16-row kernels, with a ragged last chunk and a chunk boundary at the end."""
    dtype = DTYPES[dname]
    es = torch.empty((), dtype=dtype).element_size()
    ng = D // min(D, 128 // es)
    L = chunk_rows(dtype, D, 16)
    H = 8
    B = -(-336 // (H * ng))  # at least 336 streams: 2 chunks each exceed 640
    g = torch.Generator().manual_seed(150 + D)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    for N in (L + 5, 2 * L):
        V = torch.randn(B, H, N, D, generator=g).to(dtype)
        y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
        ref, sref = O.scan(lam, V)
        assert_parity(y, ref, dtype, f"N={N} B={B}")
        assert rel_err(fin, sref) <= 1e-5, f"final state N={N}"


@pytest.mark.parametrize("dname,out", [("f32", None), ("f16", None), ("bf16", torch.float32)])
def test_scan_several_rounds(hip_device, kdecay_lib, dname, out):
    """1152 chunks of 512 rows: more than the device holds at once, so the
    launch runs in rounds; with 128 streams at most 16 chunk rows per stream
    are resident, so it takes the window-1 kernels of each type (the C4 tests
    take the window-2 ones)."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(180)
    B = 8 if dtype == torch.float32 else 16  # 128 streams (fp32 splits D=64 in two groups)
    lam = lam_uniform(8, 0.5, 0.9999, g)
    V = torch.randn(B, 8, 4100, 64, generator=g).to(dtype)
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True, out_dtype=out)
    ref, sref = O.scan(lam, V, out_dtype=out)
    assert y.dtype == (out or dtype)
    assert_parity(y, ref, out or dtype, f"{dname} rounds")
    assert rel_err(fin, sref) <= 1e-5


def test_randomized_shapes(hip_device, kdecay_lib):
    """A seeded sweep of 48 random cases against the C restatement: dtypes,
    head dims, batch and head counts on both sides of the small-grid limit,
    lengths at and around chunk boundaries, decay factors from 0.3 to 0.9999,
    contiguous V or the projection's (B,N,H*D) view, with or without a carried
    state and offset.  Outputs are compared after the reference's storage
    rounding (its zeros_like(V) output has V's dtype)."""
    rng = np.random.default_rng(2024)
    for case in range(48):
        dname = ["f32", "bf16", "f16"][rng.integers(3)]
        dtype = DTYPES[dname]
        D = int(rng.choice([16, 32, 64, 128, 256]))
        L = chunk_rows(dtype, D, int(rng.choice([8, 16])))
        B, H = int(rng.integers(1, 25)), int(rng.integers(1, 17))
        N = int(rng.choice([1, 2, int(rng.integers(3, 300)), L - 1, L, L + 1, 2 * L + int(rng.integers(-3, 4)),
                            int(rng.integers(1, 9)) * L + int(rng.integers(0, 64))]))
        N = max(1, min(N, 8_000_000 // (B * H * D) or 1))
        fused = bool(rng.integers(2))
        carry = bool(rng.integers(2))
        t_off = int(rng.integers(0, 5000)) if carry else 0
        print(f"  case {case}: {dname} B={B} H={H} N={N} D={D} fused={fused} carry={carry}", flush=True)
        g = torch.Generator().manual_seed(case)
        lam = (0.3 + (0.9999 - 0.3) * torch.rand(H, generator=g)).float()
        if fused:
            V = torch.randn(B, N, H, D, generator=g).to(dtype).transpose(1, 2)
        else:
            V = torch.randn(B, H, N, D, generator=g).to(dtype)
        init = torch.randn(B, H, D, generator=g) if carry else None
        kw = {"return_final_state": True}
        if carry:
            kw.update(initial_state=init.to(hip_device), t_offset=t_off)
        y, fin = kilat_amd.global_decay_scan(lam.to(hip_device), V.to(hip_device), **kw)
        torch.cuda.synchronize()
        ref, sref = C.scan_f32(lam.numpy(), V.float().numpy(), None if init is None else init.numpy(), t_off)
        ref = torch.from_numpy(ref).to(dtype)
        assert y.dtype == dtype and y.shape == V.shape
        assert_parity(y.cpu(), ref, dtype, f"case {case}")
        assert rel_err(fin.cpu(), torch.from_numpy(sref)) <= 1e-5, f"case {case} final state"


def test_mixed_shapes_share_one_workspace(hip_device, kdecay_lib):
    """Back-to-back launches of different shapes on one stream reuse one
    workspace: 256- and 512-row chunks, one round and several, single-chunk
    streams (no look-back) and a second dtype.  Words left by each launch,
    in layouts the next one does not share, must never be taken for its own."""
    g = torch.Generator().manual_seed(190)
    shapes = [(2, 3, 700, 64, torch.bfloat16), (16, 8, 4100, 64, torch.bfloat16),
              (4, 4, 300, 64, torch.bfloat16), (8, 8, 4100, 64, torch.float32),
              (2, 3, 200, 64, torch.bfloat16), (1, 16, 9000, 128, torch.bfloat16)]  # N=200: one chunk
    for k, (B, H, N, D, dt) in enumerate(shapes * 2):
        lam = lam_uniform(H, 0.5, 0.9999, g)
        V = torch.randn(B, H, N, D, generator=g).to(dt)
        y = gpu_scan(lam, V, hip_device)
        assert_parity(y, O.global_decay(lam, V), dt, f"launch {k} {(B, H, N, D, dt)}")
    probe = torch.empty(1, 1, 1, 64, device=hip_device)
    assert kilat_amd.workspace_error(probe) == 0


def test_many_streams_count_through_sub_counts(hip_device, kdecay_lib):
    """Launches of more than 384 streams count their last chunks toward the
    epoch's advance through 64 sub-counts; fewer streams count on one word.
    Back-to-back launches on one workspace alternate the two, twice over,
    with stream counts that are not multiples of 64 (485, 410): each launch
    must advance the epoch exactly once and leave every sub-count at zero,
    or a later launch would take older words for its own (or wait for words
    that never come, and give up).  Each is checked against the oracle,
    with carry-in and final state."""
    g = torch.Generator().manual_seed(191)
    shapes = [(97, 5, 600, 64, torch.bfloat16),   # 485 streams x 2 chunks: sub-counts
              (4, 12, 2048, 64, torch.bfloat16),  # 48 streams: one word
              (128, 12, 700, 64, torch.bfloat16),  # 1536 streams x 2 chunks
              (41, 10, 1500, 32, torch.float32)]  # 410 streams x 3 chunks
    for k, (B, H, N, D, dt) in enumerate(shapes * 2):
        lam = lam_uniform(H, 0.5, 0.9999, g)
        V = torch.randn(B, H, N, D, generator=g).to(dt)
        init = torch.randn(B, H, D, generator=g)
        y, fin = gpu_scan(lam, V, hip_device, initial_state=init.to(hip_device), return_final_state=True)
        ref, sref = C.scan_f32(lam.numpy(), V.float().numpy(), init.numpy(), 0)
        assert_parity(y.cpu(), torch.from_numpy(ref).to(dt), dt, f"launch {k} {(B, H, N, D, dt)}")
        assert rel_err(fin.cpu(), torch.from_numpy(sref)) <= 1e-5, f"launch {k} final state"
    probe = torch.empty(1, 1, 1, 64, device=hip_device)
    assert kilat_amd.workspace_error(probe) == 0


@pytest.mark.parametrize("N", [4096, 4097])
def test_chunk_size_switch(hip_device, kdecay_lib, N):
    """52 streams of bf16 D=64: N=4096 is exactly 416 chunks of 512 rows (the
    library takes 256-row chunks), N=4097 is 468 (it keeps 512-row chunks)."""
    g = torch.Generator().manual_seed(170)
    lam = lam_uniform(13, 0.5, 0.9999, g)
    V = torch.randn(4, 13, N, 64, generator=g).to(torch.bfloat16)
    ws = kdecay_lib.kdecay_scan_workspace_bytes(4, 13, N, 64, 1)
    assert ws == HDR + 4 * 13 * (16 if N == 4096 else 9) * 64 * 8
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
    ref, sref = O.scan(lam, V)
    assert_parity(y, ref, torch.bfloat16, f"N={N}")
    assert rel_err(fin, sref) <= 1e-5


@pytest.mark.parametrize("B,N,nchunk", [(20, 1024, 4), (21, 1024, 2), (10, 512, 2), (11, 512, 0)])
def test_chunk_size_switch_short_chains(hip_device, kdecay_lib, B, N, nchunk):
    """16 heads of bf16 D=64 with 2 chunks of 512 rows per stream: 640 chunks
    (B=20) take 256-row chunks, 672 (B=21) keep 512-row ones; with 1 chunk per
    stream 160 (B=10) take 256-row chunks, 176 (B=11) run without look-back.
    Against the C restatement with a carried state and an offset."""
    g = torch.Generator().manual_seed(171 + B)
    lam = lam_uniform(16, 0.5, 0.9999, g)
    V = torch.randn(B, 16, N, 64, generator=g).to(torch.bfloat16)
    init = torch.randn(B, 16, 64, generator=g)
    ws = kdecay_lib.kdecay_scan_workspace_bytes(B, 16, N, 64, 1)
    assert ws == (HDR + B * 16 * nchunk * 64 * 8 if nchunk else 0)
    y, fin = gpu_scan(lam, V, hip_device, initial_state=init.to(hip_device), return_final_state=True, t_offset=9)
    ref, sref = O.scan(lam, V, init_state=init, t_offset=9)
    assert_parity(y, ref, torch.bfloat16, f"B={B} N={N}")
    assert rel_err(fin, sref) <= 1e-5


@pytest.mark.parametrize("dname,B,H,N,D,six", [
    # one 128-byte group per head at B=1 (larger batches run as batch slices)
    ("bf16", 1, 156, 4096, 64, False),  # 1248 chunks of 512 rows: 16 rows per lane, 2 rounds
    ("bf16", 1, 168, 4096, 64, True),   # 1344: 256-row chunks, six workgroups per CU
    ("bf16", 1, 192, 4096, 64, True),   # 1536
    ("bf16", 1, 204, 4096, 64, False),  # 1632
    ("bf16", 1, 168, 4097, 64, False),  # 9 chunks per stream
    ("bf16", 1, 336, 2048, 64, True),   # 4 chunks per stream
    ("bf16", 5, 12, 4096, 128, False),  # 960 in two channel groups per head: one round
    ("bf16", 6, 12, 4096, 128, True),   # 1152
    ("f32", 8, 12, 4096, 64, True),     # 1536 in two groups of 32 fp32 channels
    ("f16", 1, 192, 4096, 64, True),
    # heads of four or more groups: 256-row chunks from 1024 chunks of 512 rows up, 32 or fewer per stream
    ("bf16", 2, 12, 4096, 256, False),  # 768: below a full round
    ("bf16", 4, 8, 4096, 256, True),    # 1024
    ("bf16", 2, 4, 16384, 256, True),   # 1024 in chains of 32
    ("bf16", 2, 4, 16896, 256, False),  # 1056 in chains of 33
    ("bf16", 8, 12, 4096, 192, False),  # three groups per head (2304)
    ("f32", 8, 12, 4096, 128, True),    # four groups of 32 fp32 channels (3072, four rounds)
])
def test_chunk_shape_just_above_one_round(hip_device, kdecay_lib, dname, B, H, N, D, six):
    """The switch to 256-row chunks at six workgroups per compute unit for
    16-row grids just above one resident round (more than 1280 chunks, or 1024
    with several channel groups per head, up to 1536, 8 or fewer per stream),
    and for heads of four or more channel groups at 1024 chunks or more with
    32 or fewer per stream, both sides of each bound, against the oracle; with
    a carried state, an offset and the final state, and for bf16 also the
    fp32 output."""
    dt = DTYPES[dname]
    es = torch.empty((), dtype=dt).element_size()
    rows = chunk_rows(dt, D, 8 if six else 16)
    ws = kdecay_lib.kdecay_scan_workspace_bytes(B, H, N, D, {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dt])
    assert ws == HDR + B * H * -(-N // rows) * D * 8, (ws, rows)
    g = torch.Generator().manual_seed(180 + B + N % 7)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dt)
    init = torch.randn(B, H, D, generator=g)
    y, fin = gpu_scan(lam, V, hip_device, initial_state=init.to(hip_device), return_final_state=True, t_offset=5)
    ref32, sref = O.scan(lam, V, init_state=init, t_offset=5, out_dtype=torch.float32)
    assert_parity(y, ref32.to(dt), dt, f"{dname} B={B} N={N} D={D}")
    assert rel_err(fin, sref) <= 1e-5
    if dt == torch.bfloat16 and es == 2:
        y32 = gpu_scan(lam, V, hip_device, initial_state=init.to(hip_device), t_offset=5, out_dtype=torch.float32)
        assert_parity(y32, ref32, torch.float32, f"{dname} fp32 out")
        assert torch.equal(y32.to(dt), y)


@pytest.mark.parametrize("dname,B,H,N,D,nslice", [
    ("bf16", 10, 12, 4096, 64, 1),   # 960 chunks of 512 rows: one launch
    ("bf16", 11, 12, 4096, 64, 2),   # 1056: batch slices of 5 and 6
    ("bf16", 17, 12, 4096, 64, 2),   # 8 + 9
    ("bf16", 48, 12, 4096, 64, 6),   # six slices of 768 chunks
    ("f16", 12, 16, 4096, 64, 2),
    ("f32", 16, 12, 4096, 32, 2),    # one 128-byte group of fp32
    ("bf16", 43, 12, 1024, 64, 2),   # 2 chunks per stream
    ("bf16", 128, 12, 512, 64, 2),   # single-chunk streams: no look-back
    ("bf16", 9, 12, 8192, 64, 1),    # 16 chunks per stream: one launch
])
def test_batch_slices(hip_device, kdecay_lib, dname, B, H, N, D, nslice):
    """Heads of one full 128-byte channel group, with at most 8 chunks of 512
    rows per stream and more than 1024 of them, run as launches over balanced
    slices of the batch, one after another on the workspace (sized for the
    largest slice); against the oracle with a carried state, an offset and
    the final state, and for bf16 also the fp32 output."""
    dt = DTYPES[dname]
    rows = chunk_rows(dt, D, 16)
    chain = -(-N // rows)
    ws = kdecay_lib.kdecay_scan_workspace_bytes(B, H, N, D, {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dt])
    assert ws == (HDR + -(-B // nslice) * H * chain * D * 8 if chain > 1 else 0), ws
    g = torch.Generator().manual_seed(230 + B + N % 7)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dt)
    init = torch.randn(B, H, D, generator=g)
    y, fin = gpu_scan(lam, V, hip_device, initial_state=init.to(hip_device), return_final_state=True, t_offset=9)
    ref, sref = C.scan_f32(lam.numpy(), V.float().numpy(), init.numpy(), 9)
    ref32 = torch.from_numpy(ref)
    assert_parity(y.cpu(), ref32.to(dt), dt, f"{dname} B={B} H={H} N={N}")
    assert rel_err(fin.cpu(), torch.from_numpy(sref)) <= 1e-5
    if dt == torch.bfloat16:
        y32 = gpu_scan(lam, V, hip_device, initial_state=init.to(hip_device), t_offset=9, out_dtype=torch.float32)
        assert_parity(y32.cpu(), ref32, torch.float32, f"{dname} fp32 out")
        assert torch.equal(y32.to(dt), y)


def test_batch_slices_replay_from_a_graph(hip_device, kdecay_lib):
    """A batch-sliced scan (B=16 H=12 N=4096: two launches on one workspace)
    captured in a HIP graph: each replay advances the epoch twice on the
    device, with eager launches of another shape on the same workspace
    between replays, and every replay equals the eager result bit for bit."""
    g = torch.Generator().manual_seed(240)
    lam = lam_uniform(12, 0.5, 0.9999, g).to(hip_device)
    V = torch.randn(16, 12, 4096, 64, generator=g).to(torch.bfloat16).to(hip_device)
    W = torch.randn(2, 12, 3000, 64, generator=g).to(torch.bfloat16).to(hip_device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        y_ref, fin_ref = kilat_amd.global_decay_scan(lam, V, return_final_state=True)  # workspace made eagerly
        w_ref = kilat_amd.global_decay_scan(lam, W)
        y = torch.empty_like(y_ref)
        fin = torch.empty_like(fin_ref)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y2, fin2 = kilat_amd.global_decay_scan(lam, V, return_final_state=True)
            y.copy_(y2)
            fin.copy_(fin2)
    torch.cuda.synchronize()
    ref, sref = C.scan_f32(lam.cpu().numpy(), V.float().cpu().numpy(), None, 0)
    assert_parity(y_ref.cpu(), torch.from_numpy(ref).to(torch.bfloat16), torch.bfloat16, "eager")
    assert rel_err(fin_ref.cpu(), torch.from_numpy(sref)) <= 1e-5
    for r in range(3):
        print(f"  graph replay {r}", flush=True)
        y.zero_(); fin.zero_()
        with torch.cuda.stream(stream):
            graph.replay()
            w = kilat_amd.global_decay_scan(lam, W)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref) and torch.equal(fin, fin_ref), r
        assert torch.equal(w, w_ref), r


def assert_same_rounding_as_fp32_output(lam, V, y, dev, ref32, what=""):
    """The scan with a 2-byte output gives bit for bit its own fp32 output
    rounded by torch (round-to-nearest-even): both are the same kernel's fp32
    values, stored once rounded and once not.  And those fp32 values meet the
    fp32 tolerance against the oracle's fp32 output (rel_err <= 1e-5 per
    stream), so the 2-byte output is one rounding of values that match the
    reference's."""
    y32 = kilat_amd.global_decay_scan(lam.to(dev), V.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert y32.dtype == torch.float32
    same = torch.equal(y.to(dev), y32.to(y.dtype))
    e = rel_err(y32, ref32)
    print(f"  {what}: 2-byte output == fp32 output rounded: {same}; fp32 output rel_err {e:.2e}", flush=True)
    assert same, what
    assert e <= 1e-5, f"{what}: fp32 output rel_err {e:.3e}"


def test_c1_fp32_full(hip_device, kdecay_lib):
    """C1 to the fp32 tolerance, read normwise per stream (max|y-ref| / max|ref|
    <= 1e-5, the gate).  The elementwise ratio |y-ref|/|ref| over elements
    with |ref| > 1e-3 max|ref| is reported beside it, with its own bound."""
    lam, V = c1_inputs()
    y = gpu_scan(lam, V, hip_device)
    ref = O.global_decay(lam, V)
    assert_parity(y, ref, torch.float32, "C1")
    emax, e9999, n = elementwise_rel(y, ref)
    # The same figures for the reference's own fp32 recurrence against exact
    # (fp64) arithmetic on the same inputs: the scale elementwise error has
    # in fp32 at all (2.3e-5 max, 1.1e-5 at the 99.99th percentile here).
    y64 = O.global_decay(lam.double(), V.double())
    rmax, r9999, _ = elementwise_rel(ref, y64)
    print(f"  C1 fp32 vs oracle: normwise {rel_err(y, ref):.3e}; elementwise over {n} elements: "
          f"max {emax:.3e}, 99.99th percentile {e9999:.3e}  (oracle vs fp64: max {rmax:.3e}, "
          f"99.99th {r9999:.3e})", flush=True)
    assert emax <= 1e-4 and e9999 <= 5e-5, (emax, e9999)


def test_c2_bf16_full(hip_device, kdecay_lib):
    """C2 to the bf16 tolerance, and its output rounding pinned: one
    round-to-nearest-even from fp32, against the oracle and against the
    kernel's own fp32 output."""
    lam, V = c2_inputs()
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
    ref32, sref = O.scan(lam, V, out_dtype=torch.float32)
    ref = ref32.to(torch.bfloat16)  # the oracle's bf16 output: the same rows rounded once
    assert_parity(y, ref, torch.bfloat16, "C2")
    assert rel_err(fin, sref) <= 1e-5
    assert kilat_amd.workspace_error(V.to(hip_device)) == 0
    assert_rounded_once(y, ref32, "C2 bf16")
    assert_same_rounding_as_fp32_output(lam, V, y, hip_device, ref32, "C2 bf16")


def test_fp16_output_rounding_c2_shape(hip_device, kdecay_lib):
    """fp16 V at the C2 shape: the same two rounding checks as C2's bf16."""
    lam, V = c2_inputs(seed=12)
    V = V.float().to(torch.float16)
    y = gpu_scan(lam, V, hip_device)
    ref32, _ = O.scan(lam, V, out_dtype=torch.float32)
    assert y.dtype == torch.float16
    assert_parity(y, ref32.to(torch.float16), torch.float16, "C2 shape fp16")
    assert_rounded_once(y, ref32, "C2 shape fp16")
    assert_same_rounding_as_fp32_output(lam, V, y, hip_device, ref32, "C2 shape fp16")


@pytest.fixture(scope="module")
def c4_oracle():
    """C4's inputs and the oracle's fp32 output and final state (65,536 steps
    on the CPU), shared by the C4 tests."""
    lam, V = c4_inputs()
    ref32, sref = O.scan(lam, V, out_dtype=torch.float32)
    return lam, V, ref32, sref


def test_c4_fp32_output_long_context(hip_device, kdecay_lib, c4_oracle):
    """C4 (D=128: two channel groups per head; 4096 chunks, several rounds)
    with an fp32 output, against the oracle's fp32 output at the fp32
    tolerance: late rows of the lam ~ 0.99999 heads are small, and only a
    tight relative check sees their carries."""
    lam, V, ref, sref = c4_oracle
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True, out_dtype=torch.float32)
    assert y.dtype == torch.float32
    assert_parity(y, ref, torch.float32, "C4 fp32 out")
    assert rel_err(fin, sref) <= 1e-5


def test_c4_bf16_long_context(hip_device, kdecay_lib, c4_oracle):
    lam, V, ref32, sref = c4_oracle
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
    ref = ref32.to(torch.bfloat16)  # the oracle's bf16 output: the same rows rounded once
    assert_parity(y, ref, torch.bfloat16, "C4")
    assert rel_err(fin, sref) <= 1e-5
    # the carry crosses 512 chunks per stream: the last rows depend on all of them
    assert max_abs(y[:, :, -4096:], ref[:, :, -4096:]) <= 2e-2
    assert_rounded_once(y, ref32, "C4 bf16")
    assert_same_rounding_as_fp32_output(lam, V, y, hip_device, ref32, "C4 bf16")


def test_sequential_kernel_matches_oracle_bits(hip_device, kdecay_lib):
    lam, V = c1_inputs(N=512)
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True, algorithm="sequential")
    ref, sref = O.scan(lam, V)
    assert torch.equal(fin.cpu(), sref)  # the recurrence itself is bit-exact
    yb = y.cpu().numpy().view(np.int32).astype(np.int64)
    rb = ref.numpy().view(np.int32).astype(np.int64)
    ulps = np.abs(yb - rb)
    assert ulps.max() <= 1 and (ulps > 0).mean() < 1e-4  # z from pow() may round one ulp apart


def test_chunked_is_deterministic(hip_device, kdecay_lib):
    lam, V = c2_inputs(B=2, N=8192)
    y1 = gpu_scan(lam, V, hip_device)
    y2 = gpu_scan(lam, V, hip_device)
    assert torch.equal(y1, y2)


def test_chunked_vs_sequential_kernel(hip_device, kdecay_lib):
    lam, V = c1_inputs(N=2000, D=32)
    y = gpu_scan(lam, V, hip_device)
    ys = gpu_scan(lam, V, hip_device, algorithm="sequential")
    assert rel_err(y, ys) <= 1e-5


@pytest.mark.parametrize("B,N,H", [(2, 700, 6), (16, 2000, 12)])
def test_layout_fused_strided_view(hip_device, kdecay_lib, B, N, H):
    """V as the (B,N,H*D) projection viewed as (B,H,N,D): no contiguous() copy
    (a small grid: 256-row chunks; and 768 chunks: 512-row chunks)."""
    g = torch.Generator().manual_seed(7)
    D = 64
    lam = lam_uniform(H, 0.8, 0.999, g)
    flat = torch.randn(B, N, H * D, generator=g).to(torch.bfloat16).to(hip_device)
    V = flat.view(B, N, H, D).transpose(1, 2)
    assert not V.is_contiguous()
    y = kilat_amd.triton_global_decay(lam.to(hip_device), V)
    assert y.stride() == V.stride()  # empty_like keeps the layout
    yc = kilat_amd.triton_global_decay(lam.to(hip_device), V.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(y, yc)
    assert_parity(y, O.global_decay(lam, V.cpu()), torch.bfloat16, "strided")


def test_misaligned_and_odd_layouts(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(8)
    lam = lam_uniform(2, 0.5, 0.99, g)
    base = torch.randn(2 * 2 * 300 * 32 + 1, generator=g)
    V = base[1:].view(2, 2, 300, 32)  # 4-byte offset: not 16-byte aligned
    y = gpu_scan(lam, V, hip_device)
    assert_parity(y, O.global_decay(lam, V), torch.float32, "misaligned")
    Vt = torch.randn(2, 2, 32, 300, generator=g).transpose(2, 3)  # d-stride != 1
    y = gpu_scan(lam, Vt, hip_device)
    assert_parity(y, O.global_decay(lam, Vt.contiguous()), torch.float32, "d-strided")


def test_unsupported_head_dim_uses_sequential_kernel(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(9)
    lam = lam_uniform(2, 0.5, 0.99, g)
    V = torch.randn(1, 2, 100, 48, generator=g)
    y = gpu_scan(lam, V, hip_device)
    assert_parity(y, O.global_decay(lam, V), torch.float32, "D=48")


@pytest.mark.parametrize("B,H", [(1, 4), (16, 8)])
def test_fp32_output_for_bf16_input(hip_device, kdecay_lib, B, H):
    lam, V = c2_inputs(B=B, N=3000, H=H)  # 24 and 768 chunks at 512 rows
    y = gpu_scan(lam, V, hip_device, out_dtype=torch.float32)
    ref, _ = O.scan(lam, V, out_dtype=torch.float32)
    assert y.dtype == torch.float32
    assert_parity(y, ref, torch.float32, "bf16->f32")


@pytest.mark.parametrize("dname", ["f32", "bf16"])
@pytest.mark.parametrize("B,H", [(2, 3), (24, 8)])
def test_chunked_prefill_with_carry(hip_device, kdecay_lib, dname, B, H):
    """Split prefill with a carried state and a position offset, on small grids
    and on grids of more than 416 chunks (the two chunk sizes)."""
    dtype = DTYPES[dname]
    lam, V = c1_inputs(B=B, N=1500, H=H, D=64)
    V = V.to(dtype)
    y, s = gpu_scan(lam, V, hip_device, return_final_state=True)
    y1, s1 = gpu_scan(lam, V[:, :, :700], hip_device, return_final_state=True)
    y2, s2 = gpu_scan(lam, V[:, :, 700:], hip_device, return_final_state=True, initial_state=s1, t_offset=700)
    ref, sref = O.scan(lam, V)
    assert_parity(torch.cat([y1, y2], 2), ref, dtype, "split")
    assert rel_err(s2, sref) <= 1e-5 and rel_err(s, sref) <= 1e-5
    r2, _ = O.scan(lam, V[:, :, 700:], init_state=s1.cpu(), t_offset=700)
    assert_parity(y2, r2, dtype, "carry-in")


def test_lambda_edges_match_oracle(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(11)
    lam = torch.tensor([0.0, 1.0, 0.5, 1e-30])
    V = torch.randn(2, 4, 2500, 16, generator=g)  # 3 chunks of 1024 rows: edges cross the carry
    V[0, 1, 0, :3] = 0.0
    y = gpu_scan(lam, V, hip_device).cpu()
    ref = O.global_decay(lam, V)
    assert torch.equal(torch.isnan(y), torch.isnan(ref))
    assert torch.equal(torch.isinf(y), torch.isinf(ref))
    fin = torch.isfinite(ref)
    assert rel_err(torch.where(fin, y, 0), torch.where(fin, ref, 0)) <= 1e-5


def test_nan_propagates_like_oracle(hip_device, kdecay_lib):
    lam, V = c1_inputs(B=1, N=900, H=2, D=64)
    V[0, 1, 300, 5] = float("nan")
    y = gpu_scan(lam, V, hip_device).cpu()
    ref = O.global_decay(lam, V)
    assert torch.equal(torch.isnan(y), torch.isnan(ref))
    assert torch.isnan(y[0, 1, 300:, 5]).all() and torch.isfinite(y[0, 1, :300]).all()


def test_triton_global_decay_signature(hip_device, kdecay_lib):
    lam, V = c1_inputs(B=1, N=300, H=2, D=32)
    y = kilat_amd.triton_global_decay(lam.to(hip_device), V.to(hip_device))
    torch.cuda.synchronize()
    assert y.dtype == V.dtype and y.shape == V.shape and y.device.type == "cuda"
    assert_parity(y, O.global_decay(lam, V), torch.float32, "drop-in")
    # lam in another float dtype is used as fp32
    y2 = kilat_amd.triton_global_decay(lam.double().to(hip_device), V.to(hip_device))
    assert torch.equal(y, y2)


def test_empty_and_degenerate(hip_device, kdecay_lib):
    lam = torch.tensor([0.9, 0.8]).to(hip_device)
    V = torch.zeros(0, 2, 10, 16, device=hip_device)
    assert kilat_amd.triton_global_decay(lam, V).shape == V.shape
    V = torch.zeros(1, 2, 0, 16, device=hip_device)
    init = torch.randn(1, 2, 16, device=hip_device)
    y, fin = kilat_amd.global_decay_scan(lam, V, initial_state=init, return_final_state=True)
    torch.cuda.synchronize()
    assert y.shape == V.shape and torch.equal(fin, init)


def test_golden_fixtures_on_gpu(hip_device, kdecay_lib):
    import os

    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "decay_golden.npz"))

    def t(name, bf16=False):
        a = d[name]
        if bf16:
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        return torch.from_numpy(a.copy())

    y, fin = gpu_scan(t("scan_f32_lam"), t("scan_f32_V"), hip_device, return_final_state=True)
    assert_parity(y, t("scan_f32_out"), torch.float32, "golden f32")
    assert rel_err(fin, t("scan_f32_final")) <= 1e-5
    y, fin = gpu_scan(t("scan_bf16_lam"), t("scan_bf16_V", True), hip_device, return_final_state=True)
    assert_parity(y, t("scan_bf16_out", True), torch.bfloat16, "golden bf16")
    y, fin = gpu_scan(t("scan_init_lam"), t("scan_init_V"), hip_device, return_final_state=True,
                      initial_state=t("scan_init_init").to(hip_device), t_offset=int(d["scan_init_offset"]))
    assert_parity(y, t("scan_init_out"), torch.float32, "golden init")
    assert rel_err(fin, t("scan_init_final")) <= 1e-5


def test_workspace_clean_after_suite(hip_device, kdecay_lib):
    lam, V = c2_inputs(B=1, N=5000, H=2)
    gpu_scan(lam, V, hip_device)
    assert kilat_amd.workspace_error(V.to(hip_device)) == 0


def test_lookback_give_up_is_flagged_not_hung(hip_device, kdecay_lib):
    """Force the bounded look-back waits to give up after one poll
    (kdecay_debug_set_spin_limit, the library's test hook): every launch still
    returns and sets the workspace's sticky error word, and the launch that
    gives up writes NaN in the rows whose carry it could not compute.  From
    then on the workspace is poisoned: every later launch on it, with the
    normal poll limit again, writes NaN to every row and to the final state
    (never finite values read from words the launch that gave up left
    behind), until the workspace is cleared; the cleared workspace serves a
    launch bit-identical to the first."""
    g = torch.Generator().manual_seed(41)
    lam = lam_uniform(16, 0.99, 0.99999, g).to(hip_device)
    V = torch.randn(1, 16, 32768, 128, generator=g).to(torch.bfloat16).to(hip_device)  # 64 chunks per stream
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        y_ref = kilat_amd.global_decay_scan(lam, V)
        torch.cuda.synchronize()
        assert kilat_amd.workspace_error(V) == 0
        kdecay_lib.kdecay_debug_set_spin_limit(1)
        gave_up = False
        try:
            for k in range(3):
                print(f"  forced give-up launch {k}", flush=True)
                y, fin = kilat_amd.global_decay_scan(lam, V, return_final_state=True)
                torch.cuda.synchronize()
                err = kilat_amd.workspace_error(V)
                if gave_up:  # the word was set before this launch: all of it NaN
                    assert bool(torch.isnan(y).all()) and bool(torch.isnan(fin).all()), k
                elif err:  # the launch that gave up: NaN, not finite wrong values
                    assert bool(torch.isnan(y).any()), k
                    gave_up = True
                else:
                    assert bool(torch.isfinite(y).all()), k
        finally:
            kdecay_lib.kdecay_debug_set_spin_limit(0)
        assert gave_up and kilat_amd.workspace_error(V) == 1
        print("  launch on the poisoned workspace", flush=True)
        y, fin = kilat_amd.global_decay_scan(lam, V, return_final_state=True)
        torch.cuda.synchronize()
        assert bool(torch.isnan(y).all()) and bool(torch.isnan(fin).all())
        assert kilat_amd.workspace_error(V) == 1
        assert kilat_amd.workspace_error(V, clear=True) == 1  # reads the word, then zeroes the workspace
        print("  launch on the cleared workspace", flush=True)
        y = kilat_amd.global_decay_scan(lam, V)
        torch.cuda.synchronize()
        assert kilat_amd.workspace_error(V) == 0
    assert torch.equal(y, y_ref) and bool(torch.isfinite(y).all())


def test_integration_ctypes_stub_matches_package(hip_device, kdecay_lib):
    """The integration guide's stand-alone ctypes stub gives the package's bits,
    on a contiguous V and on the projection's strided (B,N,H*D) view."""
    from kilat_amd import _build
    from tests.ctypes_stub import load

    stub = load(_build.LIBRARY)
    g = torch.Generator().manual_seed(43)
    lam = lam_uniform(6, 0.8, 0.999, g).to(hip_device)
    V = torch.randn(2, 6, 1500, 64, generator=g).to(torch.bfloat16).to(hip_device)
    flat = torch.randn(2, 1500, 6 * 64, generator=g).to(torch.bfloat16).to(hip_device)
    Vs = flat.view(2, 1500, 6, 64).transpose(1, 2)
    for x in (V, Vs):
        ys = stub(lam, x)
        yp = kilat_amd.triton_global_decay(lam, x)
        torch.cuda.synchronize()
        assert torch.equal(ys, yp)


def test_concurrent_streams_do_not_interfere(hip_device, kdecay_lib):
    """Scans launched on two streams at once use one workspace per stream; their
    launch epochs and look-back words must not mix.  Several interleaved rounds
    on both streams, each result against its single-stream reference."""
    g = torch.Generator().manual_seed(47)
    lam = lam_uniform(12, 0.5, 0.9999, g).to(hip_device)
    Va = torch.randn(4, 12, 4096, 64, generator=g).to(torch.bfloat16).to(hip_device)
    Vb = torch.randn(2, 12, 6000, 64, generator=g).to(torch.bfloat16).to(hip_device)
    ya_ref = kilat_amd.global_decay_scan(lam, Va)
    yb_ref = kilat_amd.global_decay_scan(lam, Vb)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    sa.wait_stream(torch.cuda.current_stream())
    sb.wait_stream(torch.cuda.current_stream())
    outs = []
    for r in range(4):
        with torch.cuda.stream(sa):
            ya = kilat_amd.global_decay_scan(lam, Va)
        with torch.cuda.stream(sb):
            yb = kilat_amd.global_decay_scan(lam, Vb)
        outs.append((ya, yb))
    torch.cuda.synchronize()
    for r, (ya, yb) in enumerate(outs):
        assert torch.equal(ya, ya_ref), r
        assert torch.equal(yb, yb_ref), r
    for s in (sa, sb):
        with torch.cuda.stream(s):
            assert kilat_amd.workspace_error(Va) == 0


def test_native_c_abi_caller(hip_device, kdecay_lib):
    """tests/c_abi_check.cpp: a C++ program that uses only include/kdecay.h and the
    HIP runtime (no Python, no torch) runs the scan, the decode step and a
    rejected argument, and checks them against its own CPU loops."""
    import os
    import subprocess

    from tests import c_abi_build

    assert os.path.exists(c_abi_build.BINARY), (
        "tests/_build/c_abi_check is missing: __graft_entry__.build() builds it next to libkdecay.so")
    print("  running tests/_build/c_abi_check", flush=True)
    r = subprocess.run([c_abi_build.BINARY], capture_output=True, text=True, timeout=60)
    print(r.stdout.strip(), flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c_abi_check OK" in r.stdout


@pytest.mark.parametrize("dname,D", [("bf16", 384), ("f32", 96), ("f32", 288), ("bf16", 48), ("f16", 8),
                                     ("f32", 1), ("bf16", 100)])
def test_scan_wide_and_padded_head_dims(hip_device, kdecay_lib, dname, D):
    """Head dims of several 128-byte channel groups (bf16 384, fp32 96 and 288)
    run on the chunked kernels as they are; others (48, 8, 1, 100) are
    zero-padded by the shim to the next head dim the kernels take.  Against
    the oracle, with a carried state and an offset, on contiguous V and on the
    projection's (B,N,H*D) view."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(260 + D)
    lam = lam_uniform(3, 0.5, 0.9999, g)
    assert kilat_amd.chunked_head_dim(D, dtype) == (D in (384, 96, 288))
    for N in (3, 1300):
        for fused in (False, True):
            if fused:
                V = torch.randn(2, N, 3, D, generator=g).to(dtype).transpose(1, 2)
            else:
                V = torch.randn(2, 3, N, D, generator=g).to(dtype)
            init = torch.randn(2, 3, D, generator=g)
            y, fin = gpu_scan(lam, V, hip_device, return_final_state=True, initial_state=init.to(hip_device),
                              t_offset=5)
            ref, sref = O.scan(lam, V, init, 5)
            assert y.shape == V.shape and y.dtype == dtype and y.stride() == V.stride()
            assert_parity(y, ref, dtype, f"D={D} N={N} fused={fused}")
            assert rel_err(fin, sref) <= 1e-5


@pytest.mark.parametrize("dname,H,N", [("bf16", 3, 2000), ("bf16", 2, 5000), ("bf16", 1, 40000), ("f32", 2, 9000),
                                       ("f16", 1, 70000), ("bf16", 6, 16128), ("bf16", 6, 16384),
                                       ("f32", 2, 16384), ("bf16", 2, 65535)])
def test_small_grid_windows(hip_device, kdecay_lib, dname, H, N):
    """Small grids (at most 416 chunks of 512 rows) of few streams with long
    chains: the one-round launch takes a look-back window of 4, 8 or 16 by
    chunks per stream (8 rows per lane: 256-row chunks for 128-byte groups),
    and from 64 such chunks per stream on (N=16384 against 16128 here) 512-row
    chunks of 8 wavefronts.  Against the C restatement at full length, with a
    carried state and an offset; the final state too."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(280 + N)
    lam = lam_uniform(H, 0.9, 0.99999, g)
    V = torch.randn(1, H, N, 64, generator=g).to(dtype)
    init = torch.randn(1, H, 64, generator=g)
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True, initial_state=init.to(hip_device), t_offset=11)
    ref, sref = C.scan_f32(lam.numpy(), V.float().numpy(), init.numpy(), 11)
    assert_parity(y.cpu(), torch.from_numpy(ref).to(dtype), dtype, f"{dname} H={H} N={N}")
    assert rel_err(fin.cpu(), torch.from_numpy(sref)) <= 1e-5
    assert kilat_amd.workspace_error(V.to(hip_device)) == 0


@pytest.mark.parametrize("dname,out,B,H,N", [("bf16", None, 8, 12, 2048), ("f32", None, 8, 12, 1024),
                                             ("bf16", torch.float32, 8, 12, 2048), ("f16", None, 4, 12, 4096)])
def test_small_grid_throttled_stores(hip_device, kdecay_lib, dname, out, B, H, N):
    """Small-grid launches (256-row chunks) with more than two workgroups per
    CU throttle their stores (768 workgroups here): one and two 16-byte stores
    per row, a ragged last chunk, against the oracle, with the final state."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(290 + N)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    for n in (N, N - 37):
        V = torch.randn(B, H, n, 64, generator=g).to(dtype)
        y, fin = gpu_scan(lam, V, hip_device, return_final_state=True, out_dtype=out)
        ref, sref = O.scan(lam, V, out_dtype=out)
        assert_parity(y, ref, out or dtype, f"{dname} N={n}")
        assert rel_err(fin, sref) <= 1e-5


# ---------------------------------------------------------------------------
# float64 V.  The reference's kernel takes any floating dtype, accumulates in
# fp32 and stores into out = empty_like(V) (triton_ops.py:149-152, 309); the
# float64 launch loads each element rounded to fp32 once, computes as the fp32
# kernels do and widens each output exactly.
# ---------------------------------------------------------------------------
def _embed_f64_groups(V64):
    """V64 rounded to fp32, each 16-channel group of the float64 head in the
    first half of a 32-channel fp32 group (zeros in the second): an fp32 launch
    with the same streams, chunks and lanes per row as the float64 one."""
    B, H, N, D = V64.shape
    V32 = torch.zeros(B, H, N, D // 16, 32, dtype=torch.float32, device=V64.device)
    V32[..., :16] = V64.float().reshape(B, H, N, D // 16, 16)
    return V32.reshape(B, H, N, 2 * D)


def _f64_channels(y32, D):
    B, H, N, _ = y32.shape
    return y32.reshape(B, H, N, D // 16, 32)[..., :16].reshape(B, H, N, D)


@pytest.mark.parametrize("B,H,N,D", [(2, 3, 3000, 16), (1, 4, 20000, 16), (2, 3, 1000, 64), (8, 12, 1100, 64),
                                     (4, 16, 2048, 48), (8, 12, 4096, 64)])
def test_scan_f64_is_the_fp32_kernel_on_rounded_input(hip_device, kdecay_lib, B, H, N, D):
    """Small grids (8 rows per lane, and the long-chain 8-wavefront kernel at
    N=20000), large grids and a 3-group head: the float64 output equals the
    fp32 kernel's on the embedded rounded input, widened, bit for bit (the
    look-back folds from the start of each stream, so equal geometry gives
    equal bits); the final states too; and y is within the fp32 bound of the
    oracle's float64 path (the reference's CPU loop in V's dtype)."""
    g = torch.Generator().manual_seed(600 + D + N)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
    assert y.dtype == torch.float64 and y.shape == V.shape
    y32, fin32 = gpu_scan(lam, _embed_f64_groups(V.to(hip_device)), hip_device, return_final_state=True)
    assert torch.equal(y, _f64_channels(y32, D).double())
    assert torch.equal(fin, _f64_channels(fin32.unsqueeze(2), D).squeeze(2))
    ref, sref = O.scan(lam, V)
    assert ref.dtype == torch.float64
    e = rel_err(y, ref)
    assert e <= 1e-5, f"float64 rel_err {e:.3e}"
    assert rel_err(fin, sref) <= 1e-5


def test_scan_f64_carry_offset_layout_and_sequential(hip_device, kdecay_lib):
    """float64 V in the projection layout ((B,N,H*D) viewed as (B,H,N,D)), with
    a carried-in state and a position offset: equal bits to the same V made
    contiguous, within the fp32 bound of the oracle; the sequential kernel on
    float64 equals the sequential kernel on V rounded to fp32, widened."""
    g = torch.Generator().manual_seed(611)
    B, H, N, D = 3, 4, 2500, 32
    lam = lam_uniform(H, 0.5, 0.9999, g)
    flat = torch.randn(B, N, H * D, generator=g, dtype=torch.float64)
    init = torch.randn(B, H, D, generator=g)
    dev = hip_device
    V = flat.to(dev).view(B, N, H, D).transpose(1, 2)
    assert not V.is_contiguous()
    kw = dict(initial_state=init.to(dev), t_offset=77, return_final_state=True)
    y, fin = gpu_scan(lam, V, dev, **kw)
    yc, finc = gpu_scan(lam, V.contiguous(), dev, **kw)
    assert y.dtype == torch.float64 and torch.equal(y, yc) and torch.equal(fin, finc)
    ref, sref = O.scan(lam, V.cpu(), init_state=init, t_offset=77)
    assert rel_err(y, ref) <= 1e-5 and rel_err(fin, sref) <= 1e-5
    ys, fins = gpu_scan(lam, V, dev, algorithm="sequential", **kw)
    ys32, fins32 = gpu_scan(lam, V.float(), dev, algorithm="sequential", **kw)
    assert ys.dtype == torch.float64 and torch.equal(ys, ys32.double()) and torch.equal(fins, fins32)
    assert rel_err(ys, ref) <= 1e-5


def test_scan_f64_rejects_float32_out_and_pads_other_head_dims(hip_device, kdecay_lib):
    """A float64 V writes float64 only (as empty_like(V)); head dims that are
    not a multiple of 16 are zero-padded like any other type's."""
    g = torch.Generator().manual_seed(612)
    lam = lam_uniform(2, 0.6, 0.999, g)
    V = torch.randn(1, 2, 700, 24, generator=g, dtype=torch.float64)
    with pytest.raises(TypeError, match="float64"):
        kilat_amd.global_decay_scan(lam.to(hip_device), V.to(hip_device), out_dtype=torch.float32)
    y = gpu_scan(lam, V, hip_device)
    assert y.dtype == torch.float64 and y.shape == V.shape
    assert rel_err(y, O.scan(lam, V)[0]) <= 1e-5


@pytest.mark.parametrize("B,H,N,D,dname", [(2, 16, 8192, 256, "bf16"), (8, 12, 4096, 128, "f32")])
def test_scan_wide_heads_several_rounds(hip_device, kdecay_lib, B, H, N, D, dname):
    """Heads of four 128-byte channel groups on grids of several rounds: the
    six-per-CU 8-row kernel in 2.7 and 4 rounds (4096 and 6144 chunks of 256
    rows), against the oracle."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(660 + D)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    y, fin = gpu_scan(lam, V, hip_device, return_final_state=True)
    ref, sref = O.scan(lam, V)
    assert_parity(y, ref, dtype, f"{dname} D={D}")
    assert rel_err(fin, sref) <= 1e-5
