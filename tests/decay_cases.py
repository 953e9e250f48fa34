"""Seeded synthetic inputs of the benchmark configurations, and error metrics.

Config numbering follows the workloads the parity tests and bench.py use:
  C1  fp32 op, B=2 N=1024 H=6 D=64, lam in [0.90, 0.999]
  C2  bf16 scan, B=8 N=4096 H=12 D=64, lam in [0.5, 0.9999], one head 0.9999
  C3  decode, 256 sequences x 12 heads x 64, random prefixes, 128 steps
  C4  bf16 long scan, B=1 N=65536 H=16 D=128, lam in [0.99, 0.99999]
"""
from __future__ import annotations

import torch

# Bytes of a scan workspace's header: launch epoch, completion count and sticky
# error word, then 64 completion sub-counts 32 bytes apart from byte 256.
WORKSPACE_HEADER_BYTES = 2304


def lam_from_uniform(u: torch.Tensor) -> torch.Tensor:
    """lam = sigmoid(log_lambda) with log_lambda = logit(u), as the layer computes it."""
    u = u.double()
    log_lambda = torch.log(u / (1 - u)).float()
    return torch.sigmoid(log_lambda)


def lam_uniform(H: int, lo: float, hi: float, g: torch.Generator) -> torch.Tensor:
    return lam_from_uniform(lo + (hi - lo) * torch.rand(H, generator=g, dtype=torch.float64))


def c1_inputs(seed: int = 0, B=2, N=1024, H=6, D=64):
    g = torch.Generator().manual_seed(seed)
    V = torch.randn(B, H, N, D, generator=g, dtype=torch.float32)
    lam = lam_uniform(H, 0.90, 0.999, g)
    return lam, V


def c2_inputs(seed: int = 1, B=8, N=4096, H=12, D=64):
    g = torch.Generator().manual_seed(seed)
    V = torch.randn(B, H, N, D, generator=g, dtype=torch.float32).to(torch.bfloat16)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    lam[H - 1] = 0.9999  # fp32 0.99989998: the long-memory head
    return lam, V


def c4_inputs(seed: int = 3, B=1, N=65536, H=16, D=128):
    g = torch.Generator().manual_seed(seed)
    V = torch.randn(B, H, N, D, generator=g, dtype=torch.float32).to(torch.bfloat16)
    lam = lam_uniform(H, 0.99, 0.99999, g)
    return lam, V


def c3_inputs(seed: int = 2, S=256, H=12, D=64, steps=128, max_prefix=2048):
    """Prefix lengths, bf16 prefix values (list, one [1,H,L,D] each), lam, bf16 step inputs [steps,S,H,D]."""
    g = torch.Generator().manual_seed(seed)
    lam = lam_uniform(H, 0.5, 0.9999, g)
    lengths = torch.randint(1, max_prefix + 1, (S,), generator=g)
    prefixes = [torch.randn(1, H, int(L), D, generator=g).to(torch.bfloat16) for L in lengths]
    v_steps = torch.randn(steps, S, H, D, generator=g).to(torch.bfloat16)
    return lam, lengths, prefixes, v_steps


def rel_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    """max over (b,h) streams of max|y - ref| / max|ref| (fp64, finite refs)."""
    y = y.double().cpu()
    ref = ref.double().cpu()
    B, H = ref.shape[:2]
    num = (y - ref).abs().reshape(B, H, -1).amax(-1)
    den = ref.abs().reshape(B, H, -1).amax(-1).clamp_min(1e-30)
    return float((num / den).max())


def elementwise_rel(y: torch.Tensor, ref: torch.Tensor, floor: float = 1e-3):
    """Elementwise |y - ref| / |ref| over the elements with |ref| > floor * max|ref|
    (fp64): returns (max, 99.99th percentile, elements counted).  Near a zero
    crossing of y the ratio is dominated by rounding of the partial sums, in
    the reference's own recurrence as much as in any reassociated one; the
    floor leaves those elements out."""
    y = y.double().cpu().reshape(-1)
    ref = ref.double().cpu().reshape(-1)
    keep = ref.abs() > floor * float(ref.abs().max())
    r = ((y - ref).abs() / ref.abs())[keep]
    if r.numel() == 0:
        return 0.0, 0.0, 0
    q = float(torch.quantile(r, 0.9999)) if r.numel() <= 1 << 24 else float(r.sort().values[int(0.9999 * (r.numel() - 1))])
    return float(r.max()), q, int(r.numel())


def max_abs(y: torch.Tensor, ref: torch.Tensor) -> float:
    return float((y.double().cpu() - ref.double().cpu()).abs().max())


def algorithmic_bytes(B, H, N, D, in_bytes, out_bytes) -> int:
    return B * H * N * D * (in_bytes + out_bytes)


def ordered_bits(x: torch.Tensor) -> torch.Tensor:
    """2-byte floats as integers in the order of their values: adjacent
    representable values (one ulp apart, across zero too) differ by 1."""
    b = x.contiguous().view(torch.int16).to(torch.int32)
    mag = b & 0x7FFF
    return torch.where(b < 0, -mag, mag)


def assert_rounded_once(y, ref32, what=""):
    """The 2-byte output y against the oracle's fp32 output rounded once to
    y's dtype, round-to-nearest-even, as the reference stores it
    (out = zeros_like(V), triton_ops.py:240,246).

    The kernel's fp32 values differ from the oracle's by reassociation: a few
    fp32 ulps of the partial sums, i.e. an absolute error of order 1e-7 of the
    stream's scale.  Rounded, that moves an element across a rounding
    boundary of the 2-byte type only rarely: at most 1e-3 of the elements may
    differ, and each by exactly one ulp of that type, except in the band
    |ref| <= 1e-3 max|ref| of its (b,h) stream, where one ulp of a small value
    is finer than that absolute error (such elements stay within the parity
    tolerance, checked apart).  A truncating store, or a second rounding,
    would miss on about half the elements."""
    r = ref32.to(y.dtype)
    d = (ordered_bits(y.cpu()) - ordered_bits(r)).abs()
    n_diff = int((d != 0).sum())
    frac = n_diff / d.numel()
    scale = ref32.abs().amax(dim=(-2, -1), keepdim=True)
    near_zero = ref32.abs() <= 1e-3 * scale
    far = d[~near_zero]
    far_max = int(far.max()) if far.numel() else 0
    n_band = int(((d > 1) & near_zero).sum())
    print(f"  {what}: {n_diff} of {d.numel()} elements off the oracle's rounding ({frac:.2e}); outside the "
          f"near-zero band at most {far_max} ulp; {n_band} near-zero elements more than one ulp off", flush=True)
    assert far_max <= 1, f"{what}: an element {far_max} ulps from the oracle's rounding"
    assert frac <= 1e-3, f"{what}: {frac:.2e} of the elements off the oracle's rounding"
