"""kilat_amd — MI355X (gfx950) global-decay scan for Kilat.

A drop-in for the global-decay path of Kilat's hybrid attention: the
full-sequence scan ``triton_global_decay`` (/root/reference/src/kilat/arc/
triton_ops.py:249) and the incremental decode update (/root/reference/src/
kilat/arc/attention.py:344-360), as hand-written HIP kernels in libkdecay.so
behind a C ABI (include/kdecay.h).
"""
from .triton_ops import (
    chunked_head_dim,
    decay_step,
    global_decay_scan,
    reserve_workspace,
    triton_global_decay,
    workspace_error,
)

__version__ = "0.1.0"

__all__ = [
    "triton_global_decay",
    "decay_step",
    "global_decay_scan",
    "workspace_error",
    "reserve_workspace",
    "chunked_head_dim",
]
