"""Stacked inference weights that hold the only copy of their parameters.

Several linears that read the same input run as one GEMM in inference.  The
stacked weight is built once and each parameter is rebound as a row view of it,
so the module keeps one copy of those weights (not the parameters plus a
concatenated cache).  Optimiser steps and ``load_state_dict`` write through the
views into the stacked tensor in place; a parameter replaced by a new tensor (``.to``,
``.half``, assignment) is detected by its data pointer and the stack is rebuilt.
"""

from __future__ import annotations

import torch


def _key(params) -> tuple:
    # No version counter: once built, the parameters are views of the stack, so
    # in-place updates already land in it; only a replaced tensor needs a rebuild.
    return tuple((p.data_ptr(), p.dtype, p.device, tuple(p.shape)) for p in params)


def stacked_rows(owner: torch.nn.Module, attr: str, params: list[torch.Tensor]) -> torch.Tensor:
    """``torch.cat(params, 0)`` as one tensor whose row ranges the parameters are views of.

    The result is cached on ``owner`` under ``attr`` until a parameter changes.  It is
    created outside inference mode, so that the rebound parameters stay usable for
    training after an inference call.
    """
    cached = owner.__dict__.get(attr)
    if cached is not None and cached[0] == _key(params):
        return cached[1]
    owner.__dict__.pop(attr, None)
    with torch.inference_mode(False), torch.no_grad():
        fused = torch.cat([p.detach() for p in params], dim=0)
        off = 0
        for p in params:
            n = p.shape[0]
            p.data = fused[off:off + n]
            off += n
    owner.__dict__[attr] = (_key(params), fused)
    return fused


def drop(owner: torch.nn.Module, *attrs: str) -> None:
    """Forget cached stacks (called before a module converts or moves its parameters)."""
    for a in attrs:
        owner.__dict__.pop(a, None)
