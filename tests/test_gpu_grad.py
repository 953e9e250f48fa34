"""GPU backward of the full-sequence scan (kdecay_scan_fwd_train + kdecay_scan_bwd
through kilat_amd's autograd Function) against fp64 torch autograd through the
oracle, which restates /root/reference/src/kilat/arc/triton_ops.py:240-246 (the
reference's differentiable CPU path; its GPU path has no backward).

Tolerances: dV as the forward (fp32: rel_err <= 1e-5; bf16/fp16: max-abs
<= 2e-2 relative to the gradient's scale); dlam and d(init) (fp32
accumulation): relative error <= 1e-4.
"""
from __future__ import annotations

import pytest
import torch

import kilat_amd
from kilat_amd import _lib
from oracle import decay_oracle as O
from tests.decay_cases import lam_uniform, rel_err
from tests.decay_cases import WORKSPACE_HEADER_BYTES as HDR

pytestmark = pytest.mark.gpu

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def oracle_grads(lam, V, gy, init=None, gfin=None, t_offset=0):
    lam64 = lam.double().requires_grad_(True)
    V64 = V.double().requires_grad_(True)
    init64 = init.double().requires_grad_(True) if init is not None else None
    y, fin = O.scan(lam64, V64, init_state=init64, t_offset=t_offset)
    loss = (y * gy.double()).sum()
    if gfin is not None:
        loss = loss + (fin * gfin.double()).sum()
    loss.backward()
    return V64.grad, lam64.grad, (init64.grad if init is not None else None)


def gpu_grads(lam, V, gy, dev, init=None, gfin=None, t_offset=0):
    lam_d = lam.to(dev).requires_grad_(True)
    V_d = V.to(dev).requires_grad_(True)
    init_d = init.to(dev).requires_grad_(True) if init is not None else None
    print(f"  grad V{tuple(V.shape)} {V.dtype} init={init is not None} gfin={gfin is not None}", flush=True)
    y, fin = kilat_amd.global_decay_scan(lam_d, V_d, initial_state=init_d, return_final_state=True,
                                         t_offset=t_offset)
    loss = (y.float() * gy.to(dev).float()).sum()
    if gfin is not None:
        loss = loss + (fin * gfin.to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    return V_d.grad.cpu(), lam_d.grad.cpu(), (init_d.grad.cpu() if init is not None else None)


def rel(a, b):
    return float((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-30))


def check(dv, dl, di, rdv, rdl, rdi, dtype, what):
    if dtype == torch.float32:
        assert rel_err(dv, rdv) <= 1e-5, f"{what}: dV rel_err {rel_err(dv, rdv):.3e}"
    else:
        e = float((dv.double() - rdv).abs().max() / rdv.abs().max())
        assert e <= 2e-2, f"{what}: dV scaled max-abs {e:.3e}"
    assert rel(dl, rdl) <= 1e-4, f"{what}: dlam rel {rel(dl, rdl):.3e}"
    if rdi is not None:
        assert rel(di, rdi) <= 1e-4, f"{what}: dinit rel {rel(di, rdi):.3e}"


@pytest.mark.parametrize("dname", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
def test_backward_shapes(hip_device, kdecay_lib, dname, D):
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(200 + D)
    lam = lam_uniform(3, 0.5, 0.999, g)
    for N in (1, 77, 300, 1100):
        V = torch.randn(2, 3, N, D, generator=g).to(dtype)
        gy = torch.randn(2, 3, N, D, generator=g).to(dtype)
        dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
        rdv, rdl, _ = oracle_grads(lam, V, gy)
        assert dv.dtype == dtype
        check(dv, dl, None, rdv, rdl, None, dtype, f"D={D} N={N}")


@pytest.mark.parametrize("dname,H,D", [("f32", 4, 64), ("bf16", 2, 128), ("bf16", 2, 64)])
def test_backward_long_sequence(hip_device, kdecay_lib, dname, H, D):
    """N = 65536: 128 backward chunks of 512 rows per stream, so the reverse
    look-back runs 128 chunks deep (several rounds for f32, one round with
    the window of 8 for bf16 D=128) and each head's dlam sums 256 chunk
    partials; bf16 H=2 D=64 (a 256-chunk grid at 512 rows) takes 128-row
    chunks instead, 512 per stream, with the window of 16.  Against the fp64
    adjoint recurrence (oracle.decay_oracle.scan_grads_f64)."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(210 + D)
    lam = lam_uniform(H, 0.9, 0.9999, g)
    N = 65536
    V = torch.randn(1, H, N, D, generator=g).to(dtype)
    gy = torch.randn(1, H, N, D, generator=g).to(dtype)
    dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
    rdv, rdl, _ = O.scan_grads_f64(lam, V, gy)
    assert dv.dtype == dtype
    check(dv, dl, None, rdv, rdl, None, dtype, f"N={N} D={D} {dname}")


@pytest.mark.parametrize("B,H,N", [(2, 4, 16384), (16, 16, 1024)])
def test_backward_give_up_is_flagged_not_hung(hip_device, kdecay_lib, B, H, N):
    """Force the bounded waits (the training forward's look-back, the
    backward's reverse look-back and its wait for a head's dlam partials) to
    give up after one poll, through the library's test hook: every launch
    still returns and sets the workspace's sticky error word, and the launch
    that gives up leaves NaN in the gradients it could not compute.  From then
    on the workspace is poisoned: the next training pass on it, with the
    normal poll limit again, gives NaN for every element of dV and for every
    head's dlam, until the workspace is cleared; the cleared workspace gives
    finite gradients bit-identical to the first run.  8 streams (each stream's
    first chunk counts toward the epoch's advance) and 256 (the head-summing
    workgroups and the last of each XCD count)."""
    g = torch.Generator().manual_seed(43)
    lam = lam_uniform(H, 0.9, 0.9999, g)
    V = torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16)  # 128 or 2 backward chunks per stream
    gy = torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        dv0, dl0, _ = gpu_grads(lam, V, gy, hip_device)
        probe = V[:, :, :1].to(hip_device)  # selects the workspace of this device and stream
        assert kilat_amd.workspace_error(probe) == 0
        kdecay_lib.kdecay_debug_set_spin_limit(1)
        gave_up = False
        try:
            for k in range(3):
                print(f"  forced give-up backward {k}", flush=True)
                dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
                torch.cuda.synchronize()
                err = kilat_amd.workspace_error(probe)
                if gave_up:  # the word was set before this pass: all of it NaN
                    assert bool(torch.isnan(dv).all()) and bool(torch.isnan(dl).all()), k
                elif err:  # the pass that gave up: NaN where it could not compute
                    assert bool(torch.isnan(dv).any()) or bool(torch.isnan(dl).any()), k
                    gave_up = True
        finally:
            kdecay_lib.kdecay_debug_set_spin_limit(0)
        assert gave_up and kilat_amd.workspace_error(probe) == 1
        dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
        assert bool(torch.isnan(dv).all()) and bool(torch.isnan(dl).all())
        assert kilat_amd.workspace_error(probe, clear=True) == 1  # reads the word, then zeroes the workspace
        dv1, dl1, _ = gpu_grads(lam, V, gy, hip_device)
        assert kilat_amd.workspace_error(probe) == 0
    assert torch.equal(dv1, dv0) and torch.equal(dl1, dl0)
    assert bool(torch.isfinite(dv1).all()) and bool(torch.isfinite(dl1).all())


def test_backward_epoch_counting_schemes_alternate(hip_device, kdecay_lib):
    """One workspace, backward launches that alternate between the two ways
    of counting toward the epoch's advance: 384 streams of 2 chunks (the
    head-summing workgroups and the last of each XCD count), 24 streams of 6
    (each stream's first chunk), 256 streams of 1 chunk, each against the
    fp64 adjoint recurrence, then the first shape again, bit-identical."""
    cases = [(24, 16, 1024), (2, 12, 3000), (16, 16, 512)]
    data = []
    for k, (B, H, N) in enumerate(cases):
        g = torch.Generator().manual_seed(220 + k)
        lam = lam_uniform(H, 0.8, 0.9999, g)
        V = torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16)
        gy = torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16)
        data.append((lam, V, gy))
    first = None
    for k in (0, 1, 2, 0):
        lam, V, gy = data[k]
        dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
        if k == 0 and first is not None:
            assert torch.equal(dv, first[0]) and torch.equal(dl, first[1])
            continue
        rdv, rdl, _ = O.scan_grads_f64(lam, V, gy)
        check(dv, dl, None, rdv, rdl, None, torch.bfloat16, f"case {k}")
        if k == 0:
            first = (dv, dl)


def test_backward_randomized(hip_device, kdecay_lib):
    """A seeded sweep of 24 random backward cases against the fp64 adjoint
    recurrence: dtypes, head dims, grids on both sides of the forward's
    small-grid limit, lengths around 128-row chunks, decay factors from 0.3
    to 0.9999, with or without carry-in, final-state gradient and offset."""
    import numpy as np

    rng = np.random.default_rng(4048)
    for case in range(24):
        dname = ["f32", "bf16", "f16"][rng.integers(3)]
        dtype = DTYPES[dname]
        D = int(rng.choice([16, 32, 64, 128, 256]))
        B, H = int(rng.integers(1, 13)), int(rng.integers(1, 9))
        N = int(rng.choice([1, 127, 128, 129, int(rng.integers(2, 3000)), 128 * int(rng.integers(2, 20)) + int(rng.integers(-2, 3))]))
        N = max(1, min(N, 3_000_000 // (B * H * D) or 1))
        extra = bool(rng.integers(2))
        print(f"  bwd case {case}: {dname} B={B} H={H} N={N} D={D} extra={extra}", flush=True)
        g = torch.Generator().manual_seed(500 + case)
        lam = (0.3 + (0.9999 - 0.3) * torch.rand(H, generator=g)).float()
        V = torch.randn(B, H, N, D, generator=g).to(dtype)
        gy = torch.randn(B, H, N, D, generator=g).to(dtype)
        init = torch.randn(B, H, D, generator=g) if extra else None
        gfin = torch.randn(B, H, D, generator=g) if extra else None
        t_off = int(rng.integers(0, 3000)) if extra else 0
        dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=t_off)
        rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=t_off)
        check(dv, dl, di, rdv, rdl, rdi if extra else None, dtype, f"case {case}")


def test_backward_init_final_offset(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(210)
    lam = lam_uniform(4, 0.8, 0.9999, g)
    V = torch.randn(2, 4, 1500, 64, generator=g)
    gy = torch.randn(2, 4, 1500, 64, generator=g)
    init = torch.randn(2, 4, 64, generator=g)
    gfin = torch.randn(2, 4, 64, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=9)
    rdv, rdl, rdi = oracle_grads(lam, V, gy, init=init, gfin=gfin, t_offset=9)
    check(dv, dl, di, rdv, rdl, rdi, torch.float32, "init+gfin+offset")


@pytest.mark.parametrize("dname,N", [("f32", 2600), ("bf16", 2600), ("bf16", 2560)])
def test_backward_init_final_offset_large_grid(hip_device, kdecay_lib, dname, N):
    """Carry-in state, final-state gradient and position offset on grids of
    more than 512 forward chunks at 512 rows (576 bf16, 1152 f32: the 16-row
    forward kernel) and 2016/4032 backward chunks, against the fp64 adjoint
    recurrence.  N = 2600 ends inside a lane's rows (the guarded loops);
    N = 2560 (five 512-row backward chunks per stream, 480 in all: the 16-row
    backward kernel) ends on a lane's last row, where the forward writes the
    final state and the backward adds its gradient on the unguarded loops."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(212)
    B, H, D = 12, 8, 64
    lam = lam_uniform(H, 0.8, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    gy = torch.randn(B, H, N, D, generator=g).to(dtype)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=33)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=33)
    check(dv, dl, di, rdv, rdl, rdi, dtype, f"large grid {dname} N={N}")


@pytest.mark.parametrize("dname,B,H,N,D", [("bf16", 4, 12, 4096, 128), ("f16", 3, 8, 3000, 256),
                                             ("bf16", 3, 12, 4100, 128)])
def test_backward_whole_row_streams(hip_device, kdecay_lib, dname, B, H, N, D):
    """Heads of 128 or 256 bf16/fp16 channels on large grids with short chains:
    the backward takes whole 256-byte rows per stream (16 lanes per row,
    256-row chunks; 768, 576 and 612 chunks here), while the forward keeps
    128-byte groups, so the saved chunk states are read by head and channel.
    N = 3000 and 4100 end inside a chunk.  Carry-in, final-state gradient and
    offset, against the fp64 adjoint recurrence."""
    dtype = DTYPES[dname]
    code = {"bf16": _lib.KDECAY_BF16, "f16": _lib.KDECAY_F16}[dname]
    nst, nch = B * H * (D // 128), (N + 255) // 256  # one stream per 128 channels, 256-row chunks
    assert kdecay_lib.kdecay_scan_bwd_workspace_bytes(B, H, N, D, code) == \
        HDR + nst * nch * 128 * 8 + (nst * nch * 8 + 255) // 256 * 256
    g = torch.Generator().manual_seed(230 + D + N)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    gy = torch.randn(B, H, N, D, generator=g).to(dtype)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    print(f"  whole-row backward {dname} {B}x{H}x{N}x{D}", flush=True)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=21)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=21)
    check(dv, dl, di, rdv, rdl, rdi, dtype, f"whole rows {dname} {B}x{H}x{N}x{D}")


@pytest.mark.parametrize("dname,B,H,N,D", [("bf16", 8, 12, 2048, 64), ("bf16", 8, 12, 2049, 64),
                                             ("f16", 8, 14, 2048, 64), ("f32", 4, 12, 2048, 64),
                                             ("bf16", 8, 12, 4096, 32)])
def test_backward_short_chain_grids(hip_device, kdecay_lib, dname, B, H, N, D):
    """Grids of 320-448 chunks at 512 rows (1024 for D=32): with chains of at
    most 4 chunks up to 384 of them the backward takes 128-row chunks (1536
    workgroups, more than one round), otherwise 512-row ones (N=2049: chains
    of 5; H=14: 448 chunks).  Carry-in state, final-state gradient and a
    position offset, against the fp64 adjoint recurrence."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(216 + H + N % 7)
    lam = lam_uniform(H, 0.7, 0.9999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    gy = torch.randn(B, H, N, D, generator=g).to(dtype)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=5)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=5)
    check(dv, dl, di, rdv, rdl, rdi, dtype, f"{dname} {B}x{H}x{N}x{D}")


def test_backward_fp32_lambda_near_one(hip_device, kdecay_lib):
    """fp32 with a decay factor within 1e-4 of 1 (a random parity sweep's case:
    B=24 H=2 N=347 D=16, V the projection's (B,N,H*D) view).  The normaliser
    1 - lam^(t+1), evaluated in fp32 as the reference's torch expression does,
    loses up to about 1e-3 relative precision at small t there, so the
    gradients of the reference's own fp32 path (torch autograd through the
    fp32 restatement of triton_ops.py:240-246) differ from the fp64 adjoint
    by about 6e-5 normwise.  The kernel follows the fp32 path: dV within 1e-6
    of it (normwise per stream), and within 2e-4 of fp64; dlam within 1e-4
    of fp64."""
    g = torch.Generator().manual_seed(10642)
    B, H, N, D = 24, 2, 347, 16
    lam = (0.3 + (0.99995 - 0.3) * torch.rand(H, generator=g)).float()
    assert float(lam.max()) > 0.9999
    V = torch.randn(B, N, H, D, generator=g).transpose(1, 2)
    gy = torch.randn(B, H, N, D, generator=g)
    dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
    rdv, rdl, _ = O.scan_grads_f64(lam, V, gy)
    lam32 = lam.clone().requires_grad_(True)
    V32 = V.clone().requires_grad_(True)
    y32, _ = O.scan(lam32, V32)
    (y32 * gy).sum().backward()
    e32, e64, ref64 = rel_err(dv, V32.grad), rel_err(dv, rdv), rel_err(V32.grad, rdv)
    print(f"  dV vs fp32 path {e32:.3e}, vs fp64 {e64:.3e} (fp32 path vs fp64 {ref64:.3e})", flush=True)
    assert e32 <= 1e-6, f"dV vs the fp32 reference path: {e32:.3e}"
    assert e64 <= 2e-4, f"dV vs fp64: {e64:.3e}"
    assert rel(dl, rdl) <= 1e-4, f"dlam rel {rel(dl, rdl):.3e}"


def test_backward_dlam_one_head_many_terms(hip_device, kdecay_lib):
    """dlam of a single head summed over 45 x 1388 x 128 = 8 M terms of both
    signs (bf16, a random parity sweep's case): its value, -2.636, is a small
    remainder of the terms, so the sums' precision decides its digits.  The
    reference's fp32 path is 1.3e-4 off the fp64 adjoint here.  This grid
    (270 chunks of 512 rows) takes 256-row chunks (8 rows per lane): 9.4e-5
    off, with the chunk partials, wavefront and workgroup sums in double (in
    fp32 they were 1.9e-4 off).  What remains is the lanes' fp32 states and
    row sums over their rows: 4 rows per lane measured 1.9e-6, 16 rows
    2.2e-4.  Bound: no worse than the reference's fp32 path."""
    B, H, N, D = 45, 1, 1388, 128
    g = torch.Generator().manual_seed(937 + 50000)
    lam = (0.3 + (0.9999 - 0.3) * torch.rand(H, generator=g)).float()
    V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    gy = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    print(f"  dlam over one head: bf16 {B}x{H}x{N}x{D}", flush=True)
    dv, dl, _ = gpu_grads(lam, V, gy, hip_device)
    rdv, rdl, _ = O.scan_grads_f64(lam, V, gy)
    assert rel(dl, rdl) <= 1.3e-4, f"dlam rel {rel(dl, rdl):.3e}"
    check(dv, dl, None, rdv, rdl, None, torch.bfloat16, "one head")


def test_backward_dlam_cancellation(hip_device, kdecay_lib):
    """dlam as a difference of two nearly equal sums (a random parity sweep's
    case: bf16 B=3 H=1 N=1534 D=128 with carry-in, final-state gradient and
    offset 834; the upstream gradient contributes 13.51 to dlam, the
    final-state gradient -12.55, in fp64).  A fixed relative bound on the
    total does not hold for any fp32 evaluation there: the reference's own
    fp32 path (torch autograd through the fp32 restatement of
    triton_ops.py:240-246) is 1.1e-3 off fp64.  The kernel must be no less
    accurate than that path (it measured 3.8e-4); dV to the bf16 bound."""
    g = torch.Generator().manual_seed(50159)
    B, H, N, D, t_off = 3, 1, 1534, 128, 834
    lam = (0.3 + (0.9999 - 0.3) * torch.rand(H, generator=g)).float()
    V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    gy = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=t_off)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=t_off)
    l32 = lam.clone().requires_grad_(True)
    V32 = V.float().requires_grad_(True)
    i32 = init.clone().requires_grad_(True)
    y32, f32 = O.scan(l32, V32, init_state=i32, t_offset=t_off)
    ((y32 * gy.float()).sum() + (f32 * gfin).sum()).backward()
    e_gpu, e_ref = rel(dl, rdl), rel(l32.grad, rdl)
    print(f"  dlam vs fp64: kernel {e_gpu:.3e}, reference fp32 path {e_ref:.3e}", flush=True)
    assert e_ref > 1e-4  # the case is as ill-conditioned as described
    assert e_gpu <= e_ref, f"dlam {e_gpu:.3e} vs the fp32 path's {e_ref:.3e}"
    e = float((dv.double() - rdv).abs().max() / rdv.abs().max())
    assert e <= 2e-2, f"dV scaled max-abs {e:.3e}"
    assert rel(di, rdi) <= 1e-4, f"dinit rel {rel(di, rdi):.3e}"


def test_backward_c1_shape_and_drop_in(hip_device, kdecay_lib):
    """C1 (B=2 N=1024 H=6 D=64 fp32) through triton_global_decay, as a training step calls it."""
    g = torch.Generator().manual_seed(211)
    log_lambda = torch.log(torch.tensor(0.9 / 0.1)) + 0.5 * torch.randn(6, generator=g)
    V = torch.randn(2, 6, 1024, 64, generator=g)
    gy = torch.randn(2, 6, 1024, 64, generator=g)
    ll = log_lambda.to(hip_device).requires_grad_(True)
    Vd = V.to(hip_device).requires_grad_(True)
    y = kilat_amd.triton_global_decay(torch.sigmoid(ll), Vd)
    (y * gy.to(hip_device)).sum().backward()
    torch.cuda.synchronize()
    ll64 = log_lambda.double().requires_grad_(True)
    V64 = V.double().requires_grad_(True)
    (O.global_decay(torch.sigmoid(ll64), V64) * gy.double()).sum().backward()
    assert rel_err(Vd.grad.cpu(), V64.grad) <= 1e-5
    assert rel(ll.grad.cpu(), ll64.grad) <= 1e-4


def test_backward_is_deterministic(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(212)
    lam = lam_uniform(3, 0.5, 0.999, g)
    V = torch.randn(2, 3, 3000, 64, generator=g).to(torch.bfloat16)
    gy = torch.randn(2, 3, 3000, 64, generator=g).to(torch.bfloat16)
    a = gpu_grads(lam, V, gy, hip_device)
    b = gpu_grads(lam, V, gy, hip_device)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_no_grad_path_unchanged(hip_device, kdecay_lib):
    """Without requires_grad the inference scan runs (no states are saved)."""
    g = torch.Generator().manual_seed(213)
    lam = lam_uniform(2, 0.5, 0.99, g).to(hip_device)
    V = torch.randn(1, 2, 700, 64, generator=g).to(hip_device)
    y = kilat_amd.triton_global_decay(lam, V)
    assert y.grad_fn is None
    Vg = V.clone().requires_grad_(True)
    y2 = kilat_amd.triton_global_decay(lam, Vg)
    torch.cuda.synchronize()
    assert y2.grad_fn is not None and torch.equal(y, y2.detach())


@pytest.mark.parametrize("N", [100, 3000])
def test_graph_capture_backward_replays(hip_device, kdecay_lib, N):
    """kdecay_scan_fwd_train + kdecay_scan_bwd captured in a HIP graph: the
    backward's dlam partials are tagged with the workspace's launch epoch, so
    every replay, with eager launches on the same workspace between replays,
    must reproduce the eager dV, dlam and d(init) bit for bit.  N=100 is one
    chunk per stream (no look-back, the epoch still advances); N=3000 is 24."""
    from kilat_amd import _lib
    from kilat_amd.triton_ops import _stream_ptr, _workspace

    lib = kdecay_lib
    g = torch.Generator().manual_seed(31)
    B, H, D = 2, 4, 64
    code = _lib.KDECAY_BF16
    lam = lam_uniform(H, 0.5, 0.999, g).to(hip_device)
    V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(hip_device)
    gy = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(hip_device)
    init = torch.randn(B, H, D, generator=g).to(hip_device)
    gfin = torch.randn(B, H, D, generator=g).to(hip_device)
    st = _lib.strides4(V.stride())
    nst = lib.kdecay_scan_saved_states_floats(B, H, N, D, code)
    y = torch.empty_like(V)
    states = torch.empty(max(nst, 1), device=hip_device)
    fin = torch.empty(B, H, D, device=hip_device)
    dV = torch.empty_like(V)
    dlam = torch.empty(H, device=hip_device)
    dinit = torch.empty(B, H, D, device=hip_device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())

    def launch():
        s = _stream_ptr(hip_device)
        nbytes = max(lib.kdecay_scan_workspace_bytes(B, H, N, D, code),
                     lib.kdecay_scan_bwd_workspace_bytes(B, H, N, D, code))
        ws = _workspace(hip_device, s, nbytes)
        wp, wn = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
        _lib.check(lib.kdecay_scan_fwd_train(V.data_ptr(), code, st, y.data_ptr(), code, st, lam.data_ptr(),
                                             init.data_ptr(), fin.data_ptr(), states.data_ptr() if nst else None,
                                             nst, B, H, N, D, 5, wp, wn, s), "fwd_train")
        _lib.check(lib.kdecay_scan_bwd(V.data_ptr(), code, st, gy.data_ptr(), st, dV.data_ptr(), st, lam.data_ptr(),
                                       init.data_ptr(), states.data_ptr() if nst else None, gfin.data_ptr(),
                                       dlam.data_ptr(), dinit.data_ptr(), B, H, N, D, 5, wp, wn, s), "bwd")

    with torch.cuda.stream(stream):
        launch()  # eager first: creates the workspace outside the capture
    torch.cuda.synchronize()
    ref = (dV.clone(), dlam.clone(), dinit.clone())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            launch()
    torch.cuda.synchronize()
    for r in range(4):
        print(f"  backward graph replay {r} N={N}", flush=True)
        dV.zero_(); dlam.zero_(); dinit.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dV, ref[0]) and torch.equal(dlam, ref[1]) and torch.equal(dinit, ref[2]), r
        with torch.cuda.stream(stream):
            launch()
        torch.cuda.synchronize()
        assert torch.equal(dlam, ref[1]), r
    with torch.cuda.stream(stream):
        assert kilat_amd.workspace_error(V) == 0


@pytest.mark.parametrize("dname,D", [("f32", 1), ("f32", 48), ("bf16", 8), ("bf16", 48), ("bf16", 96), ("f16", 100),
                                     ("f32", 96), ("bf16", 384), ("f32", 288)])
def test_backward_any_head_dim(hip_device, kdecay_lib, dname, D):
    """Every head dim has a backward (the reference's CPU path is differentiable
    for any D): dims the chunked kernels do not take are zero-padded in a
    differentiable way; 384 (bf16) and 288 (fp32) exercise heads of several
    128-byte channel groups beyond 256.  With a carried state, a final-state
    gradient and an offset."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(230 + D)
    lam = lam_uniform(3, 0.5, 0.999, g)
    for N in (5, 700):
        V = torch.randn(2, 3, N, D, generator=g).to(dtype)
        gy = torch.randn(2, 3, N, D, generator=g).to(dtype)
        init = torch.randn(2, 3, D, generator=g)
        gfin = torch.randn(2, 3, D, generator=g)
        dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=9)
        rdv, rdl, rdi = oracle_grads(lam, V, gy, init=init, gfin=gfin, t_offset=9)
        assert dv.shape == V.shape and dv.dtype == dtype
        check(dv, dl, di, rdv, rdl, rdi, dtype, f"D={D} N={N}")


@pytest.mark.parametrize("D", [64, 40])
def test_backward_sequential_and_out(hip_device, kdecay_lib, D):
    """algorithm='sequential' and out= keep their forward results (the
    sequential kernel's bits; the given tensor filled) and still carry the
    backward, against fp64 autograd through the oracle."""
    g = torch.Generator().manual_seed(240 + D)
    lam = lam_uniform(4, 0.5, 0.999, g)
    V = torch.randn(2, 4, 900, D, generator=g)
    gy = torch.randn(2, 4, 900, D, generator=g)
    rdv, rdl, _ = oracle_grads(lam, V, gy)
    y_seq_nograd = kilat_amd.global_decay_scan(lam.to(hip_device), V.to(hip_device), algorithm="sequential")
    for kw in ({"algorithm": "sequential"}, {"out": "given"}):
        lam_d = lam.to(hip_device).requires_grad_(True)
        V_d = V.to(hip_device).requires_grad_(True)
        out = None
        if kw.get("out") == "given":
            out = torch.empty(V.shape, device=hip_device)
            kw = {"out": out}
        print(f"  grad D={D} {list(kw)}", flush=True)
        y = kilat_amd.global_decay_scan(lam_d, V_d, **kw)
        if out is not None:
            assert y is out
        else:
            assert torch.equal(y.detach(), y_seq_nograd)
        (y * gy.to(hip_device)).sum().backward()
        torch.cuda.synchronize()
        check(V_d.grad.cpu(), lam_d.grad.cpu(), None, rdv, rdl, None, torch.float32, f"D={D} {list(kw)}")


@pytest.mark.parametrize("B,N", [(8, 2600), (2, 700)])
def test_backward_layout_fused_and_broadcast_gradient(hip_device, kdecay_lib, B, N):
    """V as the attention's projection output [B,N,H*D] viewed as [B,H,N,D]
    (row stride H*D, no copy) and the loss y.sum(), whose upstream gradient
    is a broadcast tensor of ones (every stride 0): the 512-row backward
    (B=8: 384 chunks, the tail chunk 40 rows long) and the 128-row one (B=2),
    against the fp64 adjoint recurrence."""
    H, D = 8, 64
    g = torch.Generator().manual_seed(214 + B)
    lam = lam_uniform(H, 0.8, 0.9999, g)
    proj = torch.randn(B, N, H * D, generator=g).to(torch.bfloat16)
    P = proj.to(hip_device).requires_grad_(True)
    Vd = P.view(B, N, H, D).transpose(1, 2)
    assert Vd.stride(2) == H * D
    lam_d = lam.to(hip_device).requires_grad_(True)
    print(f"  fused-layout grad B={B} N={N}", flush=True)
    y = kilat_amd.global_decay_scan(lam_d, Vd)
    y.sum().backward()
    torch.cuda.synchronize()
    V = proj.view(B, N, H, D).transpose(1, 2).contiguous()
    rdv, rdl, _ = O.scan_grads_f64(lam, V, torch.ones(B, H, N, D, dtype=torch.float64))
    dv = P.grad.cpu().view(B, N, H, D).transpose(1, 2)
    check(dv, lam_d.grad.cpu(), None, rdv, rdl, None, torch.bfloat16, f"fused layout B={B} N={N}")


def test_backward_float64_runs_the_fp32_kernels(hip_device, kdecay_lib):
    """A float64 V with a gradient runs the fp32 training forward and backward
    on V rounded to fp32: y, dV and dlam equal those of the same call on
    V.float() (widened to float64 where V's type is float64), and are within
    the fp32 bounds of the oracle's float64 gradients."""
    g = torch.Generator().manual_seed(650)
    B, H, N, D = 2, 3, 1500, 64
    dev = hip_device
    lam = lam_uniform(H, 0.6, 0.999, g)
    V = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    gy = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    Vd, ld = V.to(dev).requires_grad_(True), lam.to(dev).requires_grad_(True)
    y = kilat_amd.triton_global_decay(ld, Vd)
    assert y.dtype == torch.float64
    (y * gy.to(dev)).sum().backward()
    V32, l32 = V.float().to(dev).requires_grad_(True), lam.to(dev).requires_grad_(True)
    y32 = kilat_amd.triton_global_decay(l32, V32)
    (y32 * gy.float().to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert Vd.grad.dtype == torch.float64
    assert torch.equal(y, y32.double()) and torch.equal(Vd.grad, V32.grad.double()) and torch.equal(ld.grad, l32.grad)
    rdv, rdl, _ = oracle_grads(lam, V, gy)
    assert rel_err(Vd.grad.cpu(), rdv) <= 1e-5
    assert rel(ld.grad.cpu(), rdl) <= 1e-4


@pytest.mark.parametrize("B,H,N,D,dname", [(5, 12, 4096, 64, "f32"), (1, 16, 16384, 128, "f32"),
                                           (1, 12, 16384, 256, "bf16")])
def test_backward_256_row_chunks_of_multi_group_heads(hip_device, kdecay_lib, B, H, N, D, dname):
    """Heads of two or more 128-byte channel groups on more than one round of
    512-row chunks with at least 48 streams take 256-row chunks (8 rows per
    lane) in several rounds: fp32 D=64 (1920 chunks), fp32 D=128 with chains
    of 64, bf16 D=256 on 128-byte groups (chains of 64); against the
    oracle's float64 adjoint recurrence, with carry-in, final-state gradient
    and offset."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(700 + D + B)
    lam = lam_uniform(H, 0.5, 0.999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    gy = torch.randn(B, H, N, D, generator=g).to(dtype)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    assert _lib.load().kdecay_scan_bwd_workspace_bytes(B, H, N, D, {torch.float32: _lib.KDECAY_F32,
                                                                      torch.bfloat16: _lib.KDECAY_BF16}[dtype]) > 0
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=37)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=37)
    check(dv, dl, di, rdv, rdl, rdi, dtype, f"{dname} B={B} H={H} N={N} D={D}")


def test_backward_after_training_forward_of_many_streams(hip_device, kdecay_lib):
    """A training forward of 485 streams (more than 384: its last chunks
    count through the workspace's sub-counts) saves the states its backward
    starts from; both against the oracle's float64 adjoint, twice in a row
    on the same workspaces, with carry-in, final-state gradient and offset."""
    g = torch.Generator().manual_seed(720)
    B, H, N, D = 97, 5, 600, 64
    for rep in range(2):
        lam = lam_uniform(H, 0.5, 0.999, g)
        V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
        gy = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
        init = torch.randn(B, H, D, generator=g)
        gfin = torch.randn(B, H, D, generator=g)
        dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=11)
        rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=11)
        check(dv, dl, di, rdv, rdl, rdi, torch.bfloat16, f"rep {rep} B={B} H={H} N={N} D={D}")


@pytest.mark.parametrize("B,H,N,dname", [(11, 12, 4096, "bf16"), (43, 12, 1024, "bf16")])
def test_backward_after_batch_sliced_training_forward(hip_device, kdecay_lib, B, H, N, dname):
    """A training forward that runs as two batch slices (more than 1024
    chunks of 512 rows of one-group heads) saves each slice's states where
    the whole batch's backward reads them, and the first slice alone writes
    the per-row terms; against the oracle's float64 adjoint, with carry-in,
    final-state gradient and offset."""
    dtype = DTYPES[dname]
    g = torch.Generator().manual_seed(740 + B)
    lam = lam_uniform(H, 0.5, 0.999, g)
    V = torch.randn(B, H, N, 64, generator=g).to(dtype)
    gy = torch.randn(B, H, N, 64, generator=g).to(dtype)
    init = torch.randn(B, H, 64, generator=g)
    gfin = torch.randn(B, H, 64, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=21)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=21)
    check(dv, dl, di, rdv, rdl, rdi, dtype, f"{dname} B={B} H={H} N={N}")


def test_backward_in_two_batch_slices_matches_oracle(hip_device, kdecay_lib):
    """One-group heads whose backward grid is exactly two resident rounds
    (B=16 H=12 N=4096: 2 x 768 chunks of 512 rows) run as two launches over
    halves of the batch, the second adding the first one's dlam sums in
    double; against the oracle's float64 adjoint, with carry-in, final-state
    gradient and offset."""
    B, H, N, D = 16, 12, 4096, 64
    assert _lib.load().kdecay_scan_bwd_workspace_bytes(B, H, N, D, _lib.KDECAY_BF16) > \
        _lib.load().kdecay_scan_bwd_workspace_bytes(B // 2, H, N, D, _lib.KDECAY_BF16)
    g = torch.Generator().manual_seed(760)
    lam = lam_uniform(H, 0.5, 0.999, g)
    V = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    gy = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=3)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=3)
    check(dv, dl, di, rdv, rdl, rdi, torch.bfloat16, f"B={B} H={H} N={N}")


def test_backward_batch_slices_equal_separate_launches(hip_device, kdecay_lib):
    """B=24 H=12 N=4096 (3 x 768 chunks) runs as three backward launches of 8
    batch elements each: dV and d(init) bit for bit those of three separate
    training passes over the same thirds of the batch (each one launch of 768
    chunks), and dlam their sum, to the parts' fp32 rounding."""
    B, H, N, D = 24, 12, 4096, 64
    g = torch.Generator(device=hip_device).manual_seed(770)
    lam = (0.5 + 0.499 * torch.rand(H, generator=g, device=hip_device)).float()
    V = torch.randn(B, H, N, D, generator=g, device=hip_device).to(torch.bfloat16)
    gy = torch.randn(B, H, N, D, generator=g, device=hip_device).to(torch.bfloat16)
    init = torch.randn(B, H, D, generator=g, device=hip_device)
    gfin = torch.randn(B, H, D, generator=g, device=hip_device)

    def grads(b0, b1):
        lam_d = lam.clone().requires_grad_(True)
        V_d = V[b0:b1].clone().requires_grad_(True)
        i_d = init[b0:b1].clone().requires_grad_(True)
        y, fin = kilat_amd.global_decay_scan(lam_d, V_d, initial_state=i_d, return_final_state=True, t_offset=7)
        ((y.float() * gy[b0:b1].float()).sum() + (fin * gfin[b0:b1]).sum()).backward()
        torch.cuda.synchronize()
        return V_d.grad, lam_d.grad.double(), i_d.grad

    print("  grad V(24, 12, 4096, 64) in three slices, then three separate thirds", flush=True)
    dv, dl, di = grads(0, B)
    parts = [grads(b0, b0 + 8) for b0 in (0, 8, 16)]
    assert torch.equal(dv, torch.cat([p[0] for p in parts]))
    assert torch.equal(di, torch.cat([p[2] for p in parts]))
    dl_sum = parts[0][1] + parts[1][1] + parts[2][1]
    scale = parts[0][1].abs() + parts[1][1].abs() + parts[2][1].abs()  # each part is rounded to fp32 once
    assert bool(((dl.double() - dl_sum).abs() <= 1e-6 * scale).all()), (dl, dl_sum)


@pytest.mark.parametrize("B,H,N,D,dname", [(8, 12, 2048, 64, "bf16"), (1, 16, 8192, 64, "bf16"),
                                           (4, 12, 2048, 64, "f32")])
def test_backward_one_round_of_256_row_chunks(hip_device, kdecay_lib, B, H, N, D, dname):
    """Grids of more than 192 and at most 512 chunks of 512 rows (128-byte
    groups) take 256-row chunks in one round: bf16 at 384 chunks, at 256 in
    chains of 32 (the window-8 kernel), and fp32 with two groups per head;
    against the oracle's float64 adjoint recurrence, with carry-in,
    final-state gradient and offset."""
    dtype = DTYPES[dname]
    code = {torch.float32: _lib.KDECAY_F32, torch.bfloat16: _lib.KDECAY_BF16}[dtype]
    nst = B * H * (D * torch.empty((), dtype=dtype).element_size() // 128)
    # the workspace holds one look-back word per channel per 256-row chunk
    nch = -(-N // 256)
    assert _lib.load().kdecay_scan_bwd_workspace_bytes(B, H, N, D, code) == \
        HDR + B * H * nch * D * 8 + (nst * nch * 8 + 255) // 256 * 256
    g = torch.Generator().manual_seed(720 + B + N)
    lam = lam_uniform(H, 0.5, 0.999, g)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    gy = torch.randn(B, H, N, D, generator=g).to(dtype)
    init = torch.randn(B, H, D, generator=g)
    gfin = torch.randn(B, H, D, generator=g)
    dv, dl, di = gpu_grads(lam, V, gy, hip_device, init=init, gfin=gfin, t_offset=11)
    rdv, rdl, rdi = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=11)
    check(dv, dl, di, rdv, rdl, rdi, dtype, f"{dname} B={B} H={H} N={N} D={D}")
