"""Write tests/golden/decay_golden.npz: small input/output vectors of the oracle.

The vectors come from oracle/decay_oracle.py (the restatement of the
reference's CPU path), after tests/test_oracle.py has pinned it against
closed forms, an fp64 brute force and the independent C restatement.  They
freeze today's bits so a later torch or oracle change that moves them shows up
as a fixture failure, and they give the GPU tests cases with known answers.
bf16 tensors are stored as their uint16 bit patterns.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import decay_oracle as O  # noqa: E402
from tests.decay_cases import lam_uniform  # noqa: E402

OUT = os.path.join(HERE, "decay_golden.npz")


def bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def make() -> dict:
    g = torch.Generator().manual_seed(2024)
    d = {}

    # fp32 scan, several chunks' worth of rows for the small kernels' shapes
    lam = lam_uniform(3, 0.9, 0.999, g)
    V = torch.randn(2, 3, 40, 16, generator=g)
    out, fin = O.scan(lam, V)
    d.update(scan_f32_lam=bits(lam), scan_f32_V=bits(V), scan_f32_out=bits(out), scan_f32_final=bits(fin))

    # bf16 scan with the lam ~ 1 head
    lam = lam_uniform(2, 0.5, 0.9999, g)
    lam[1] = 0.9999
    V = torch.randn(1, 2, 70, 32, generator=g).to(torch.bfloat16)
    out, fin = O.scan(lam, V)
    d.update(scan_bf16_lam=bits(lam), scan_bf16_V=bits(V), scan_bf16_out=bits(out), scan_bf16_final=bits(fin))

    # carry-in state and position offset (chunked prefill)
    lam = lam_uniform(2, 0.8, 0.99, g)
    V = torch.randn(2, 2, 24, 16, generator=g)
    init = torch.randn(2, 2, 16, generator=g)
    out, fin = O.scan(lam, V, init_state=init, t_offset=5)
    d.update(scan_init_lam=bits(lam), scan_init_V=bits(V), scan_init_init=bits(init),
             scan_init_out=bits(out), scan_init_final=bits(fin), scan_init_offset=np.int64(5))

    # edge lambdas: 0 (no memory), 1 (z = 0: inf/nan), 0.5
    lam = torch.tensor([0.0, 1.0, 0.5])
    V = torch.randn(1, 3, 6, 16, generator=g)
    V[0, 1, 0, :4] = 0.0
    out, fin = O.scan(lam, V)
    d.update(edge_lam=bits(lam), edge_V=bits(V), edge_out=bits(out), edge_final=bits(fin))

    # decode step: scalar t_pos (reference) and per-sequence t_pos
    lam = lam_uniform(3, 0.5, 0.9999, g)
    state = torch.randn(4, 3, 16, generator=g) * 5
    v = torch.randn(4, 3, 16, generator=g).to(torch.bfloat16)
    out, ns = O.step(lam, state, v, 7)
    tpos = [0, 1, 2, 1000]
    out2, ns2 = O.step(lam, state, v, tpos)
    d.update(step_lam=bits(lam), step_state=bits(state), step_v=bits(v), step_tpos_scalar=np.int64(7),
             step_out=bits(out), step_new_state=bits(ns), step_tpos=np.array(tpos, np.int64),
             step_out_vec=bits(out2), step_new_state_vec=bits(ns2))
    return d


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(OUT, os.path.getsize(OUT), "bytes")
