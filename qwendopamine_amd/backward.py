"""Chunkwise gdn2 backward on the HIP backend (placeholder until the kernels land)."""

from __future__ import annotations


def chunk_gdn2_bwd(*args, **kwargs):
    raise NotImplementedError("chunk_gdn2 backward: HIP kernels not built yet")
