"""CPU oracle of Kilat's global-decay path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline).  The
product (kilat_amd) never calls it.

Each function restates the reference's CPU code with the same torch
operations in the same order, so on the same torch build it produces the
reference's bits:

  scan / global_decay   /root/reference/src/kilat/arc/triton_ops.py:232-247
  step                  /root/reference/src/kilat/arc/attention.py:344-360
  seed_state            /root/reference/src/kilat/arc/attention.py:383-394
  scan_grads_f64        the gradients torch autograd takes through
                        triton_ops.py:240-246, by the adjoint recurrence in
                        float64 (for sequences too long for autograd's graph)

The reference itself is never imported.  What pins these restatements
(tests/test_oracle.py): closed forms (constant input, impulse, N=1), an fp64
dense brute force, bit-equality with the independent C restatement in
oracle/decay_oracle.c, cross-function identities (step == scan, seed ==
scan's final state) and the committed fixtures in tests/golden/.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def scan(
    lam: torch.Tensor,
    V: torch.Tensor,
    init_state: Optional[torch.Tensor] = None,
    t_offset: int = 0,
    out_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """triton_ops.py:232-247, extended with a carry-in state and a position offset.

    With init_state=None and t_offset=0 it is the reference's loop verbatim:
        state = lam_b * state + V[:, :, t, :]
        z     = (1.0 - lam_b ** (t + 1)) / (1.0 - lam_b + 1e-6)
        out[:, :, t, :] = state / z
    Returns (out, final state).  `out` has V's dtype unless out_dtype is given
    (the reference's zeros_like(V) rounds each stored row to V's dtype).
    """
    B, H, N, D = V.shape
    out = torch.zeros_like(V, dtype=out_dtype or V.dtype)
    lam_b = lam.view(1, H, 1)
    if init_state is None:
        state = torch.zeros(B, H, D, device=V.device, dtype=V.dtype)
    else:
        state = init_state.clone()
    for t in range(N):
        state = lam_b * state + V[:, :, t, :]
        z = (1.0 - lam_b ** (t_offset + t + 1)) / (1.0 - lam_b + 1e-6)
        out[:, :, t, :] = state / z
    return out, state


def global_decay(lam: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """The reference's _cpu_global_decay(lam, V) (triton_ops.py:232-247)."""
    return scan(lam, V)[0]


def step(
    lam: torch.Tensor,
    past_state: torch.Tensor,
    v_current: torch.Tensor,
    t_pos,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """attention.py:344-360: one incremental step; returns (out, new_state).

    t_pos is an int shared by the batch (the reference: the latent cache
    length), or a sequence of B ints (per-sequence positions, an extension):
    each row then uses the reference's scalar expression with its own t_pos.
    """
    H = lam.shape[0]
    lam_bc = lam.view(1, H, 1)
    new_state = lam_bc * past_state + v_current
    if isinstance(t_pos, int):
        z_inc = (1 - lam_bc ** (t_pos + 1)) / (1 - lam_bc + 1e-6)
        return new_state / z_inc, new_state
    rows = []
    for b, tp in enumerate(t_pos):
        z_inc = (1 - lam_bc ** (int(tp) + 1)) / (1 - lam_bc + 1e-6)
        rows.append(new_state[b : b + 1] / z_inc)
    return torch.cat(rows, 0), new_state


def seed_state(lam: torch.Tensor, V_global: torch.Tensor, x_dtype: torch.dtype) -> torch.Tensor:
    """attention.py:383-394: the decode cache's state after a full-sequence pass."""
    B, H, N, Dh = V_global.shape
    lam_bc = lam.view(1, H, 1)
    acc_state = torch.zeros(B, H, Dh, device=V_global.device, dtype=x_dtype)
    for t in range(N):
        acc_state = lam_bc * acc_state + V_global[:, :, t, :]
    return acc_state


def scan_grads_f64(
    lam: torch.Tensor,
    V: torch.Tensor,
    gy: torch.Tensor,
    init_state: Optional[torch.Tensor] = None,
    gfin: Optional[torch.Tensor] = None,
    t_offset: int = 0,
):
    """Gradients of sum(y * gy) (+ sum(final_state * gfin)) for (y, final_state)
    = scan(lam, V, init_state, t_offset), in float64: (dV, dlam, d(init)).

    The derivative of triton_ops.py:240-246 that autograd computes, written as
    the adjoint recurrence, so that it runs at lengths autograd's graph cannot
    hold.  With s_t = lam s_{t-1} + V_t, y_t = s_t / z_t and
    z_t = (1 - lam^e) / ((1 - lam) + 1e-6), e = t_offset + t + 1:
        g_t    = gy_t / z_t + lam g_{t+1}   (+ gfin at t = N-1),  dV_t = g_t
        dlam   = sum_t g_t s_{t-1} + sum_t gy_t s_t d(1/z_t)/dlam
        d(init) = lam g_0
    with d(1/z)/dlam = (e lam^(e-1) ((1 - lam) + 1e-6) - (1 - lam^e)) / (1 - lam^e)^2.
    dlam is summed over batch and channels per head.
    """
    import numpy as np

    B, H, N, D = V.shape
    f64 = torch.float64
    l = lam.detach().to("cpu", f64).numpy().reshape(1, H, 1)
    # Time-major float64 copies (torch does the big elementwise work; the two
    # recurrences step through contiguous rows in numpy).
    v = V.detach().to("cpu", f64).permute(2, 0, 1, 3).contiguous().numpy()
    g_y = gy.detach().to("cpu", f64).permute(2, 0, 1, 3).contiguous()
    s = np.zeros((N + 1, B, H, D))  # s[t + 1] = s_t; s[0] = initial state
    if init_state is not None:
        s[0] = init_state.detach().to("cpu", f64).numpy()
    for t in range(N):
        s[t + 1] = l * s[t] + v[t]
    e = (t_offset + torch.arange(N, dtype=f64) + 1).view(N, 1, 1, 1)
    l4 = torch.from_numpy(l).view(1, 1, H, 1)
    p = l4 ** e
    den = (1.0 - l4) + 1e-6
    z = (1.0 - p) / den
    dinvz = (e * l4 ** (e - 1) * den - (1.0 - p)) / (1.0 - p) ** 2
    u = (g_y / z).numpy()
    if gfin is not None:
        u[N - 1] += gfin.detach().to("cpu", f64).numpy()
    dv = np.empty_like(u)
    g = np.zeros((B, H, D))
    for t in range(N - 1, -1, -1):
        g = u[t] + l * g
        dv[t] = g
    st = torch.from_numpy(s)
    dvt = torch.from_numpy(dv)
    dlam = (dvt * st[:N]).sum(dim=(0, 1, 3)) + (g_y * st[1:] * dinvz).sum(dim=(0, 1, 3))
    dinit = torch.from_numpy(l * dv[0])
    return dvt.permute(1, 2, 0, 3).contiguous(), dlam, dinit
