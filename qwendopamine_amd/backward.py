"""Chunkwise gdn2 backward on the HIP backend.

``chunk_gdn2_bwd`` replaces the reference ``chunk_gdn2_bwd`` and the gradient
mapping of ``ChunkGDN2Function.backward`` (``chunk_gdn2.py:2170-2325`` and
``:2480-2547``): one call of ``gdn2_chunk_bwd`` (a reverse state scan and a
chunk-parallel kernel, ``csrc/gdn2_chunk_bwd.hip``) on the training
workspace the forward filled.  There is no CPU path.
"""

from __future__ import annotations

import torch

from . import _native as nat


def chunk_gdn2_bwd(saved: dict, do: torch.Tensor, dht: torch.Tensor | None, has_h0: bool):
    """Gradients ``(dq, dk, dv, dg, db, dw, dh0)`` w.r.t. the kernel inputs.

    ``saved`` is what ``ops.chunk_gdn2_fwd(..., save_for_bwd=True)`` returned;
    ``dq, dk, dv, db, dw`` come back in the inputs' dtype, ``dg`` in g's dtype,
    ``dh0`` (float32) only when the forward had an initial state.
    """
    q, k, v, g, b, w = (saved[n] for n in ("q", "k", "v", "g", "b", "w"))
    B, T, H, K = q.shape
    V = v.shape[-1]
    N = saved["N"]
    dt = q.dtype
    if do is None:
        do = torch.zeros_like(v)
    do = do.to(dt).contiguous()
    if do.data_ptr() % 16:
        do = do.clone()
    sk = (V, K) if saved.get("transpose") else (K, V)
    dht = None if dht is None else dht.float().contiguous()
    if dht is not None and tuple(dht.shape) != (N, H, *sk):
        raise ValueError(f"chunk_gdn2 backward: dht must be {(N, H, *sk)}, got {tuple(dht.shape)}")
    dq, dk, db = torch.empty_like(q), torch.empty_like(k), torch.empty_like(b)
    dv, dw = torch.empty_like(v), torch.empty_like(w)
    dg = torch.empty_like(g)
    dh0 = torch.empty(N, H, *sk, dtype=torch.float32, device=q.device) if has_h0 else None
    lib = nat.load()
    cu_host = saved["cu_host"]
    cu_host_p = None if cu_host is None else cu_host.data_ptr()
    ws_bytes = lib.gdn2_chunk_bwd_workspace_size(B, T, H, K, V, nat.dtype_code(dt), cu_host_p, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    sv = saved["ws"]
    st = lib.gdn2_chunk_bwd(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(g), nat.ptr(b), nat.ptr(w),
        nat.dtype_code(dt), nat.dtype_code(g.dtype), nat.ptr(do), nat.ptr(dht),
        nat.ptr(dq), nat.ptr(dk), nat.ptr(dv), nat.ptr(dg), nat.ptr(db), nat.ptr(dw), nat.ptr(dh0),
        nat.ptr(saved["cu_dev"]), cu_host_p, N, B, T, H, K, V, saved["scale"], saved["flags"],
        sv.data_ptr(), sv.numel(), ws.data_ptr(), ws.numel(), nat.stream_handle(q.device),
    )
    nat.check(st, "chunk_gdn2 backward")
    return dq, dk, dv, dg, db, dw, dh0
