"""Swap Kilat's full-sequence decay op for the MI355X one, by name.

Kilat binds the op by name into its attention module
(/root/reference/src/kilat/arc/attention.py:6, ``from .triton_ops import
triton_global_decay``) and re-exports it (/root/reference/src/kilat/arc/
__init__.py:6), so a swap has to replace the attribute in every module that
holds it, not only in ``kilat.arc.triton_ops``.

The installed function is ``kilat_amd.triton_global_decay``: HIP tensors only.
A CPU tensor raises instead of being computed on the host, so a model that runs
on the CPU must not be patched (it keeps Kilat's own function).

The incremental update and the decode-state seed loop are inline code in
``KilatAttention.forward`` (attention.py:344-360, :383-394) and cannot be
swapped by name; their replacements are ``kilat_amd.decay_step`` and
``kilat_amd.global_decay_scan(..., return_final_state=True)``.
"""
from __future__ import annotations

import types
from typing import Dict, Iterable

from .triton_ops import triton_global_decay

# Modules of the reference package that hold the op by name.
KILAT_MODULES = ("kilat.arc.triton_ops", "kilat.arc.attention", "kilat.arc")

_ATTR = "triton_global_decay"


def install(modules: Iterable[types.ModuleType]) -> Dict[types.ModuleType, object]:
    """Point each module's ``triton_global_decay`` at the MI355X op.

    Returns {module: previous function} for ``uninstall``.  A module without
    the attribute raises AttributeError (nothing is patched then).
    """
    modules = list(modules)
    for m in modules:
        if not hasattr(m, _ATTR):
            raise AttributeError(f"kilat_amd.integration: {m.__name__} has no {_ATTR}")
    previous = {}
    for m in modules:
        previous[m] = getattr(m, _ATTR)
        setattr(m, _ATTR, triton_global_decay)
    return previous


def install_into_kilat() -> Dict[types.ModuleType, object]:
    """``install`` on Kilat's own modules (they must be importable)."""
    import importlib

    return install(importlib.import_module(name) for name in KILAT_MODULES)


def uninstall(previous: Dict[types.ModuleType, object]) -> None:
    """Restore what ``install`` replaced."""
    for m, fn in previous.items():
        setattr(m, _ATTR, fn)
