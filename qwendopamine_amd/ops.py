"""Kernel-level gdn2 ops on the MI355X HIP backend.

Mirrors the reference op interfaces so callers can swap them in unchanged:

* ``fused_recurrent_gdn2`` / ``fused_recurrent_gdn2_fwd`` -- reference
  ``models/gdn2/gdn2_ops/fused_recurrent_gdn2.py:461-555`` / ``:344-458``
  (token-serial forward: decode steps and short prefills, inference only).
* ``chunk_gdn2`` (+ ``ChunkGDN2Function``) -- reference
  ``models/gdn2/gdn2_ops/chunk_gdn2.py:1268-1434`` / ``:2328-2547``
  (chunkwise prefill and training forward/backward).

Both run the hand-written kernels of ``libgdn2_hip.so`` on the current HIP
stream of the inputs' device.  Like the reference ops (``chunk_gdn2.py:1267``,
``fused_recurrent_gdn2.py:344``), the public ops are excluded from
``torch.compile`` tracing (``torch.compiler.disable``): a compiled caller breaks
its graph around them and runs them eagerly.  Inputs must be ROCm GPU tensors: there is no
CPU path, and a missing library raises.  Semantics follow the reference
oracle ``torch_recurrent_gdn2`` (``gdn2.py:100-184``); the final state is
float32 (as the reference's accelerated ops return it).
"""

from __future__ import annotations

from typing import Any

import ctypes

import torch
import torch.nn.functional as F

from . import _native as nat

__all__ = [
    "fused_recurrent_gdn2",
    "fused_recurrent_gdn2_fwd",
    "chunk_gdn2",
    "chunk_gdn2_fwd",
    "chunk_gdn2_static",
    "ChunkGDN2Function",
    "gate_activation",
    "short_convolution",
    "gated_rmsnorm",
    "rms_norm",
    "add_rms_norm",
    "silu_mul",
    "linear",
    "linear_addnorm",
    "linear_pair",
    "argmax_rows",
    "attention_decode",
    "decode_step_fused",
]


def _require_gpu(name: str, *tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{name}: the gdn2 HIP kernels need ROCm GPU tensors (got a {t.device} "
                "tensor); this package has no CPU path."
            )


def _check_shapes(name, q, k, v, g, b, w, same_heads: bool) -> None:
    """Every tensor must match the dims passed to the kernels (they index by them)."""
    if q.dim() != 4 or v.dim() != 4:
        raise ValueError(f"{name}: q and v must be 4-D [B, T, H, D]")
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    if tuple(k.shape) != (B, T, H, K):
        raise ValueError(f"{name}: k shape {tuple(k.shape)} != q shape {tuple(q.shape)}")
    if tuple(v.shape[:2]) != (B, T) or tuple(w.shape) != (B, T, HV, V):
        raise ValueError(f"{name}: v / w must be [B, T, HV, V]; got {tuple(v.shape)}, {tuple(w.shape)}")
    if tuple(g.shape) != (B, T, HV, K) or tuple(b.shape) != (B, T, HV, K):
        raise ValueError(f"{name}: g / b must be [B, T, HV, K]; got {tuple(g.shape)}, {tuple(b.shape)}")
    if HV % H != 0 or (same_heads and HV != H):
        raise ValueError(f"{name}: value heads {HV} incompatible with key heads {H}")


def _check_packed(q: torch.Tensor, initial_state: torch.Tensor | None, cu_seqlens) -> None:
    """Packed (``cu_seqlens``) calls take one row of tokens and one state per sequence."""
    if cu_seqlens is None:
        return
    if q.shape[0] != 1:
        raise ValueError(f"packed sequences (cu_seqlens) go in a single row: got batch {q.shape[0]}, "
                         "concatenate the sequences along the token axis")
    n = len(cu_seqlens) - 1
    if initial_state is not None and initial_state.shape[0] != n:
        raise ValueError(f"cu_seqlens lists {n} sequences but initial_state holds "
                         f"{initial_state.shape[0]} states")


def _flags(use_qk_l2norm_in_kernel: bool, use_gate_in_kernel: bool, lower_bound) -> int:
    f = 0
    if use_qk_l2norm_in_kernel:
        f |= nat.FLAG_L2NORM_QK
    if use_gate_in_kernel:
        f |= nat.FLAG_GATE_IN_KERNEL
        if lower_bound is not None:
            f |= nat.FLAG_LOWER_BOUND
    return f


def _io(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Contiguous copy in ``dtype``, 16-byte aligned (the kernels use 16-byte loads)."""
    x = x.to(dtype).contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _gate_tensors(use_gate_in_kernel, A_log, dt_bias, heads: int, K: int):
    """float32 device copies of the in-kernel gate parameters (A_log [heads], dt_bias [heads*K])."""
    if not use_gate_in_kernel:
        return None, None
    if A_log is None:
        raise AssertionError("use_gate_in_kernel needs the A_log keyword argument")
    a = A_log.detach().float().contiguous()
    if a.numel() != heads:
        raise ValueError(f"A_log must have {heads} elements, got {a.numel()}")
    d = None if dt_bias is None else dt_bias.detach().float().contiguous()
    if d is not None and d.numel() != heads * K:
        raise ValueError(f"dt_bias must have {heads * K} elements, got {d.numel()}")
    return a, d


def _cu(cu_seqlens, device, total_tokens: int):
    """Device and host int64 copies of ``cu_seqlens``, validated on the host.

    The kernels index tokens through these offsets, so they must start at 0,
    be non-decreasing and end at the packed length.
    """
    if cu_seqlens is None:
        return None, None
    cu_host = torch.as_tensor(cu_seqlens).detach().to("cpu", torch.int64).contiguous()
    if cu_host.dim() != 1 or cu_host.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D tensor of N+1 offsets")
    if int(cu_host[0]) != 0 or int(cu_host[-1]) != total_tokens or bool((cu_host[1:] < cu_host[:-1]).any()):
        raise ValueError(
            f"cu_seqlens must start at 0, be non-decreasing and end at {total_tokens}; "
            f"got {cu_host.tolist()[:8]}..."
        )
    cu_dev = cu_host.to(device=device)
    return cu_dev, cu_host


@torch.compiler.disable
def fused_recurrent_gdn2_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
    scale: float | None = None,
    output_final_state: bool = False,
    inplace_final_state: bool = True,
    cu_seqlens: torch.LongTensor | None = None,
    ssm_state_indices: torch.Tensor | None = None,
    num_accepted_tokens: torch.Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    lower_bound: float | None = None,
    out: torch.Tensor | None = None,
    transpose_state_layout: bool = False,
    bw_logits: bool = False,
    **kwargs: Any,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Launch the token-serial HIP kernel (reference ``fused_recurrent_gdn2.py:344-458``).

    ``bw_logits`` (an extension of this backend) passes ``b`` and ``w`` as the
    pre-activation logits; the kernel applies the sigmoid in fp32.

    Final state (as the reference resolves it, ``:395-404``):

    * ``inplace_final_state`` writes back into ``initial_state``, which must be
      float32 with contiguous ``[HV, K, V]`` rows (any row stride).
    * Otherwise ``output_final_state`` allocates a new float32 state,
      ``[N, HV, K, V]`` (``[N, HV, V, K]`` with ``transpose_state_layout``).

    Serving options (kernel ``:215-232, 311-333``):

    * ``ssm_state_indices`` (``[N]`` or ``[N, T_max]``, int32/int64) makes
      ``initial_state`` a state pool.  Sequence ``n`` starts from slot
      ``idx[n, i0]``, where ``i0 = num_accepted_tokens[n] - 1`` when speculative
      and 0 otherwise.
    * The state after each of its tokens ``t`` is stored to slot ``idx[n, t]``
      (in place), or else to row ``bos + t`` of the new final state.  That state
      has ``max(N, tokens)`` rows, so every token's row exists.
    * A negative or out-of-range slot marks a padded entry: it starts from a zero
      state and its states are not stored.
    * ``transpose_state_layout`` stores every state as ``[V, K]`` (K fastest).
    """
    name = "fused_recurrent_gdn2"
    _require_gpu(name, q, k, v, g, b, w, initial_state, ssm_state_indices, num_accepted_tokens)
    _check_shapes(name, q, k, v, g, b, w, same_heads=False)
    B, T, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    if scale is None:
        scale = K**-0.5
    dt = q.dtype
    q, k, v, b, w = (_io(x, dt) for x in (q, k, v, b, w))
    g = _io(g, g.dtype if g.dtype in (torch.float32, dt) else torch.float32)
    cu_dev, cu_host = _cu(cu_seqlens, q.device, T)
    N = B if cu_seqlens is None else cu_host.numel() - 1
    state_shape = (HV, V, K) if transpose_state_layout else (HV, K, V)
    if out is None:
        out = torch.empty_like(v)
    else:
        assert out.shape == v.shape and out.dtype == dt and out.is_contiguous()

    pooled = ssm_state_indices is not None
    idx = acc = None
    idx_stride = 0
    if pooled:
        idx = ssm_state_indices
        if idx.dtype not in (torch.int32, torch.int64):
            idx = idx.long()
        idx = idx.contiguous()
        assert idx.dim() in (1, 2) and idx.shape[0] >= N, (
            f"ssm_state_indices must be [N] or [N, T] with N >= {N}; got {tuple(idx.shape)}"
        )
        idx_stride = 1 if idx.dim() == 1 else idx.shape[1]
        if num_accepted_tokens is not None:
            acc = num_accepted_tokens
            if acc.dtype not in (torch.int32, torch.int64):
                acc = acc.long()
            acc = acc.contiguous()
            assert acc.numel() >= N, f"num_accepted_tokens needs {N} entries; got {acc.numel()}"

    def _rows(x):
        assert tuple(x.shape[1:]) == state_shape, (
            f"state rows must be {state_shape}; got {tuple(x.shape[1:])}"
        )
        assert x.stride()[1:] == (state_shape[1] * state_shape[2], state_shape[2], 1), (
            "state rows must be contiguous"
        )
        return x.shape[0], x.stride(0)

    h0 = None
    h0_rows = h0_stride = 0
    if initial_state is not None:
        if inplace_final_state:
            assert initial_state.dtype == torch.float32, (
                "inplace_final_state needs a float32 initial_state"
            )
            h0 = initial_state
        else:
            h0 = initial_state.float()
            if h0.stride()[1:] != (state_shape[1] * state_shape[2], state_shape[2], 1):
                h0 = h0.contiguous()
        h0_rows, h0_stride = _rows(h0)
        if not pooled:
            assert h0_rows == N, f"initial_state must have {N} rows; got {h0_rows}"
    if inplace_final_state:
        assert initial_state is not None, "inplace_final_state=True requires an initial_state"
        ht = h0
    elif output_final_state:
        rows = max(N, B * T) if pooled else N
        ht = torch.empty(rows, *state_shape, dtype=torch.float32, device=q.device)
    else:
        ht = None
    ht_rows, ht_stride = _rows(ht) if ht is not None else (0, 0)
    for x in (h0, ht):
        if x is not None and (x.data_ptr() % 16 or x.stride(0) % 4):
            raise ValueError(f"{name}: state rows must be 16-byte aligned")

    # Gate parameters per key head (fused_recurrent_gdn2.py:259-265).
    a_log, dtb = _gate_tensors(use_gate_in_kernel, A_log, dt_bias, H, K)
    flags = _flags(use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound)
    if transpose_state_layout:
        flags |= nat.FLAG_TRANSPOSE_STATE
    if inplace_final_state:
        flags |= nat.FLAG_INPLACE_FINAL_STATE
    if bw_logits:
        flags |= nat.FLAG_SIGMOID_BW
    lib = nat.load()
    st = lib.gdn2_recurrent_fwd_ex(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(g), nat.ptr(b), nat.ptr(w),
        nat.dtype_code(dt), nat.dtype_code(g.dtype), nat.ptr(out),
        nat.ptr(h0), h0_rows, h0_stride, nat.ptr(ht), ht_rows, ht_stride,
        nat.ptr(a_log), nat.ptr(dtb),
        float(lower_bound) if lower_bound is not None else 0.0,
        nat.ptr(cu_dev), N,
        nat.ptr(idx), nat.index_dtype_code(idx), 0 if idx is None else idx.numel(), idx_stride,
        nat.ptr(acc), nat.index_dtype_code(acc),
        B, T, H, HV, K, V, float(scale), flags,
        nat.stream_handle(q.device),
    )
    nat.check(st, name)
    return out, ht


@torch.compiler.disable
def fused_recurrent_gdn2(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    lower_bound: float | None = None,
    cu_seqlens: torch.LongTensor | None = None,
    transpose_state_layout: bool = False,
    bw_logits: bool = False,
    **kwargs: Any,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Token-by-token gdn2 forward, inference only (reference ``fused_recurrent_gdn2.py:461-555``).

    Shapes: ``q, k [B,T,H,K]``, ``v, w [B,T,HV,V]``, ``g, b [B,T,HV,K]``,
    ``initial_state [N,HV,K,V]`` float32.  Returns ``(o [B,T,HV,V], final_state)``.
    """
    _check_packed(q, initial_state, cu_seqlens)
    assert b.shape == (*q.shape[:2], v.shape[2], k.shape[-1]) or b.shape == (*q.shape[:3], k.shape[-1]), (
        f"erase gate b: expected [B, T, HV, K], got {tuple(b.shape)}"
    )
    assert w.shape == v.shape, f"write gate w: expected the shape of v {tuple(v.shape)}, got {tuple(w.shape)}"
    return fused_recurrent_gdn2_fwd(
        q=q, k=k, v=v, g=g, b=b, w=w, A_log=A_log, dt_bias=dt_bias, scale=scale,
        initial_state=initial_state, inplace_final_state=False,
        output_final_state=output_final_state,
        use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
        use_gate_in_kernel=use_gate_in_kernel, lower_bound=lower_bound,
        cu_seqlens=cu_seqlens, transpose_state_layout=transpose_state_layout, bw_logits=bw_logits,
    )


class GateFunction(torch.autograd.Function):
    """The decay gate on its HIP kernels with their VJP: ``gdn2_gate_fwd`` /
    ``gdn2_gate_bwd`` (reference ``kda_gate_fwd`` / ``kda_gate_bwd`` and
    ``KDAGateFunction``, ``chunk_kda.py:3223-3340``)."""

    @staticmethod
    def forward(ctx, g, A_log, dt_bias, lower_bound):
        name = "gate_activation"
        _require_gpu(name, g, A_log, dt_bias)
        H, K = g.shape[-2], g.shape[-1]
        dt = g.dtype if g.dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        gr = _io(g, dt)
        a = _io(A_log.reshape(-1), torch.float32)
        db = None if dt_bias is None else _io(dt_bias.reshape(-1), torch.float32)
        if a.numel() != H or (db is not None and db.numel() != H * K):
            raise ValueError(f"{name}: A_log must hold {H} values and dt_bias {H * K}, got "
                             f"{a.numel()} and {None if db is None else db.numel()}")
        flags = nat.FLAG_LOWER_BOUND if lower_bound is not None else 0
        y = torch.empty(gr.shape, dtype=torch.float32, device=g.device)
        st = nat.load().gdn2_gate_fwd(
            nat.ptr(gr), nat.dtype_code(dt), nat.ptr(a), nat.ptr(db),
            float(lower_bound) if lower_bound is not None else 0.0, flags, nat.ptr(y),
            gr.numel() // (H * K), H, K, nat.stream_handle(g.device))
        nat.check(st, name)
        ctx.save_for_backward(gr, a, db)
        ctx.meta = (lower_bound, flags, g.dtype, A_log.dtype, A_log.shape,
                    None if dt_bias is None else (dt_bias.dtype, dt_bias.shape))
        return y

    @staticmethod
    def backward(ctx, dy):
        gr, a, db = ctx.saved_tensors
        lower_bound, flags, g_dtype, a_dtype, a_shape, db_meta = ctx.meta
        H, K = gr.shape[-2], gr.shape[-1]
        tokens = gr.numel() // (H * K)
        dyc = _io(dy, torch.float32)
        dgr = torch.empty_like(gr)
        dA = torch.empty(H, dtype=torch.float32, device=gr.device)
        ddt = None if db is None else torch.empty(H * K, dtype=torch.float32, device=gr.device)
        lib = nat.load()
        ws_bytes = lib.gdn2_gate_bwd_workspace_size(tokens, H, K, int(db is not None))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=gr.device)
        st = lib.gdn2_gate_bwd(
            nat.ptr(gr), nat.dtype_code(gr.dtype), nat.ptr(a), nat.ptr(db),
            float(lower_bound) if lower_bound is not None else 0.0, flags, nat.ptr(dyc), nat.ptr(dgr),
            nat.ptr(dA), nat.ptr(ddt), tokens, H, K, ws.data_ptr(), ws.numel(), nat.stream_handle(gr.device))
        nat.check(st, "gate_activation backward")
        d_db = None if ddt is None else ddt.to(db_meta[0]).reshape(db_meta[1])
        return dgr.to(g_dtype), dA.to(a_dtype).reshape(a_shape), d_db, None


def gate_activation(g: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor | None,
                    lower_bound: float | None) -> torch.Tensor:
    """The in-kernel decay activation as a differentiable step on the HIP kernels, float32.

    ``g = -exp(A_log[h]) * softplus(g + dt_bias[h, d])``, or with a lower bound
    ``g = lower_bound * sigmoid(exp(A_log[h]) * (g + dt_bias[h, d]))``
    (reference ``kda_gate`` forward, ``chunk_kda.py:3025-3053``; the same
    formula the HIP kernels apply under ``GDN2_FLAG_GATE_IN_KERNEL``).  Its
    backward gives the gradients of ``g``, ``A_log`` and ``dt_bias``
    (``kda_gate_bwd``, ``chunk_kda.py:3254-3292``).
    """
    return GateFunction.apply(g, A_log, dt_bias, lower_bound)


def chunk_gdn2_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    scale: float,
    initial_state: torch.Tensor | None,
    output_final_state: bool,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    lower_bound: float | None = None,
    cu_seqlens: torch.LongTensor | None = None,
    save_for_bwd: bool = False,
    transpose_state_layout: bool = False,
    return_intermediate_states: bool = False,
    bw_logits: bool = False,
):
    """Launch the chunkwise HIP forward (reference ``chunk_gdn2.py:1165-1264``).

    Returns ``(o, final_state)``. Optional extras:
    * ``return_intermediate_states`` appends ``h``: each chunk's start state, ``[B, NT, H, K, V]``
      (``B = 1`` with ``cu_seqlens``, NT the total chunk count) in k's dtype (``chunk_kda.py:2257-2263``).
    * ``save_for_bwd`` appends ``saved``: the inputs as the kernels read them, plus the training
      workspace that ``chunk_gdn2_bwd`` consumes.

    ``transpose_state_layout`` makes every state ``[.., V, K]``. ``bw_logits`` passes ``b`` and
    ``w`` as the pre-activation logits, activated in-kernel (forward only: not with the
    saved training workspace).
    """
    name = "chunk_gdn2"
    _require_gpu(name, q, k, v, g, b, w, initial_state)
    _check_shapes(name, q, k, v, g, b, w, same_heads=True)
    B, T, H, K = q.shape
    V = v.shape[-1]
    dt = q.dtype
    q, k, v, b, w = (_io(x, dt) for x in (q, k, v, b, w))
    g = _io(g, g.dtype if g.dtype in (torch.float32, dt) else torch.float32)
    cu_dev, cu_host = _cu(cu_seqlens, q.device, T)
    N = B if cu_seqlens is None else cu_host.numel() - 1
    sk = (V, K) if transpose_state_layout else (K, V)
    h0 = None if initial_state is None else initial_state.float().contiguous()
    if h0 is not None and tuple(h0.shape) != (N, H, *sk):
        raise ValueError(f"{name}: initial_state must be {(N, H, *sk)}, got {tuple(h0.shape)}")
    ht = torch.empty(N, H, *sk, dtype=torch.float32, device=q.device) if output_final_state else None
    keep = save_for_bwd or return_intermediate_states
    o = torch.empty_like(v)
    lib = nat.load()
    cu_host_p = None if cu_host is None else cu_host.data_ptr()
    size_fn = lib.gdn2_chunk_train_workspace_size if keep else lib.gdn2_chunk_fwd_workspace_size
    # float32 inputs with d_k > 128 run the token-serial wide path, which needs no
    # workspace outside training (a size of 0).
    ws_bytes = size_fn(B, T, H, K, V, nat.dtype_code(dt), cu_host_p, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    a_log, dtb = _gate_tensors(use_gate_in_kernel, A_log, dt_bias, H, K)
    flags = _flags(use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound)
    if transpose_state_layout:
        flags |= nat.FLAG_TRANSPOSE_STATE
    if save_for_bwd and use_gate_in_kernel:
        raise NotImplementedError(f"{name}: apply the gate before the op when gradients are needed")
    if keep:
        flags |= nat.FLAG_SAVE_FOR_BWD
    if bw_logits:
        if keep:
            raise NotImplementedError(f"{name}: bw_logits is a forward-only option; activate b and w "
                                      "before the op when the training workspace is kept")
        flags |= nat.FLAG_SIGMOID_BW
    st = lib.gdn2_chunk_fwd(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(g), nat.ptr(b), nat.ptr(w),
        nat.dtype_code(dt), nat.dtype_code(g.dtype), nat.ptr(o),
        nat.ptr(h0), nat.ptr(ht), nat.ptr(a_log), nat.ptr(dtb),
        float(lower_bound) if lower_bound is not None else 0.0,
        nat.ptr(cu_dev), cu_host_p, N, B, T, H, K, V, float(scale), flags,
        ws.data_ptr(), ws.numel(), nat.stream_handle(q.device),
    )
    nat.check(st, name)
    res = (o, ht)
    if return_intermediate_states:
        nc = sum(-(-int(cu_host[i + 1] - cu_host[i]) // 64) for i in range(N)) if cu_host is not None \
            else B * (-(-T // 64))
        nb = 1 if cu_host is not None else B
        h = torch.empty(nb, nc // max(nb, 1), H, *sk, dtype=dt, device=q.device)
        st = lib.gdn2_chunk_states(ws.data_ptr(), ws.numel(), nat.dtype_code(dt), nat.ptr(h),
                                   int(transpose_state_layout), cu_host_p, N, B, T, H, K, V,
                                   nat.stream_handle(q.device))
        nat.check(st, name)
        res = res + (h,)
    if not save_for_bwd:
        return res
    saved = dict(q=q, k=k, v=v, g=g, b=b, w=w, ws=ws, cu_dev=cu_dev, cu_host=cu_host, N=N,
                 scale=float(scale), flags=flags & ~nat.FLAG_SAVE_FOR_BWD,
                 transpose=transpose_state_layout)
    return res + (saved,)


@torch.compiler.disable
def chunk_gdn2_static(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    out: torch.Tensor,
    final_state: torch.Tensor | None = None,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    lower_bound: float | None = None,
    cu_seqlens: torch.Tensor | None = None,
    cu_seqlens_cpu: torch.Tensor | None = None,
    transpose_state_layout: bool = False,
    bw_logits: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Chunkwise forward (inference) that allocates nothing: C entry ``gdn2_chunk_fwd_static``.

    For callers that cannot allocate device memory (graph capture, serving loops).  The
    results equal ``chunk_gdn2_fwd``'s; the per-chunk workspace is a static device array
    of ``_native.STATIC_SCRATCH_BYTES`` (72 MiB) per GPU, so larger shapes raise
    ``ValueError``.  Nothing is copied or allocated here either: ``q, k, v, b, w`` must be
    contiguous, 16-byte aligned and of one dtype, ``g`` contiguous in float32 or that dtype,
    ``out`` a contiguous tensor shaped like ``v``, the states contiguous float32
    ``[N, H, K, V]`` (``[N, H, V, K]`` transposed), ``A_log`` / ``dt_bias`` contiguous float32,
    and packed sequences need both ``cu_seqlens`` (device) and ``cu_seqlens_cpu`` (host),
    int64.  Calls that overlap on one GPU share its array and race.
    Returns ``(out, final_state)``.
    """
    name = "chunk_gdn2_static"
    _require_gpu(name, q, k, v, g, b, w, out, initial_state, final_state, A_log, dt_bias, cu_seqlens)
    _check_shapes(name, q, k, v, g, b, w, same_heads=True)
    B, T, H, K = q.shape
    V = v.shape[-1]
    dt = q.dtype
    for nm, x in (("q", q), ("k", k), ("v", v), ("b", b), ("w", w), ("out", out)):
        if x.dtype != dt or not x.is_contiguous() or x.data_ptr() % 16:
            raise ValueError(f"{name}: {nm} must be a contiguous, 16-byte aligned {dt} tensor")
    if g.dtype not in (torch.float32, dt) or not g.is_contiguous():
        raise ValueError(f"{name}: g must be contiguous float32 or {dt}")
    if out.shape != v.shape:
        raise ValueError(f"{name}: out must have the shape of v {tuple(v.shape)}")
    if (cu_seqlens is None) != (cu_seqlens_cpu is None):
        raise ValueError(f"{name}: packed sequences need both cu_seqlens and cu_seqlens_cpu")
    N = B
    if cu_seqlens is not None:
        _check_packed(q, initial_state, cu_seqlens_cpu)
        if (cu_seqlens.dtype != torch.int64 or cu_seqlens_cpu.dtype != torch.int64
                or cu_seqlens_cpu.is_cuda or not cu_seqlens.is_contiguous()
                or not cu_seqlens_cpu.is_contiguous() or cu_seqlens.numel() != cu_seqlens_cpu.numel()):
            raise ValueError(f"{name}: cu_seqlens / cu_seqlens_cpu must be contiguous int64 on the "
                             "device / host, of equal length")
        N = cu_seqlens_cpu.numel() - 1
    sk = (V, K) if transpose_state_layout else (K, V)
    for nm, x in (("initial_state", initial_state), ("final_state", final_state)):
        if x is not None and (x.dtype != torch.float32 or not x.is_contiguous()
                              or tuple(x.shape) != (N, H, *sk)):
            raise ValueError(f"{name}: {nm} must be a contiguous float32 {(N, H, *sk)} tensor")
    for nm, x in (("A_log", A_log), ("dt_bias", dt_bias)):
        if x is not None and (x.dtype != torch.float32 or not x.is_contiguous()):
            raise ValueError(f"{name}: {nm} must be contiguous float32")
    if use_gate_in_kernel and A_log is None:
        raise AssertionError("use_gate_in_kernel needs the A_log keyword argument")
    flags = _flags(use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound)
    if transpose_state_layout:
        flags |= nat.FLAG_TRANSPOSE_STATE
    if bw_logits:
        flags |= nat.FLAG_SIGMOID_BW
    if scale is None:
        scale = K**-0.5
    lib = nat.load()
    with torch.cuda.device(q.device):
        st = lib.gdn2_chunk_fwd_static(
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(g), nat.ptr(b), nat.ptr(w),
            nat.dtype_code(dt), nat.dtype_code(g.dtype), nat.ptr(out),
            nat.ptr(initial_state), nat.ptr(final_state),
            nat.ptr(A_log if use_gate_in_kernel else None), nat.ptr(dt_bias if use_gate_in_kernel else None),
            float(lower_bound) if lower_bound is not None else 0.0,
            nat.ptr(cu_seqlens), None if cu_seqlens_cpu is None else cu_seqlens_cpu.data_ptr(), N,
            B, T, H, K, V, float(scale), flags, nat.stream_handle(q.device),
        )
    nat.check(st, name)
    return out, final_state


class ChunkGDN2Function(torch.autograd.Function):
    """Autograd wrapper of the chunkwise HIP kernels (reference ``chunk_gdn2.py:2328-2547``).

    The training forward keeps its workspace (per-chunk blobs, chunk start
    states and values, sequence end states) instead of recomputing them in
    backward: MI355X has the HBM for it.
    """

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, A_log, dt_bias, scale, initial_state, output_final_state,
                use_qk_l2norm_in_kernel, use_gate_in_kernel, cu_seqlens, lower_bound,
                transpose_state_layout=False):
        needs = any(ctx.needs_input_grad[i] for i in (0, 1, 2, 3, 4, 5, 9))
        if use_gate_in_kernel and needs:
            raise NotImplementedError(
                "chunk_gdn2: gradients through the in-kernel gate are taken by applying the gate "
                "before the op (chunk_gdn2 does this itself)"
            )
        res = chunk_gdn2_fwd(
            q, k, v, g, b, w, scale, initial_state, output_final_state,
            use_qk_l2norm_in_kernel, use_gate_in_kernel, A_log, dt_bias, lower_bound, cu_seqlens,
            save_for_bwd=needs, transpose_state_layout=transpose_state_layout,
        )
        ctx.in_dtypes = tuple(x.dtype for x in (q, k, v, g, b, w))
        ctx.has_h0 = initial_state is not None
        ctx.saved = res[-1] if needs else None
        return res[0], res[1]

    @staticmethod
    def backward(ctx, do, dht):
        from .backward import chunk_gdn2_bwd

        if ctx.saved is None:
            raise RuntimeError("chunk_gdn2: backward called without a training forward")
        dq, dk, dv, dg, db, dw, dh0 = chunk_gdn2_bwd(ctx.saved, do, dht, ctx.has_h0)
        ctx.saved = None
        dq, dk, dv, dg, db, dw = (x.to(d) for x, d in zip((dq, dk, dv, dg, db, dw), ctx.in_dtypes))
        return (dq, dk, dv, dg, db, dw, None, None, None, dh0, None, None, None, None, None, None)


@torch.compiler.disable
def chunk_gdn2(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    cu_seqlens: torch.LongTensor | None = None,
    cu_seqlens_cpu: torch.LongTensor | None = None,
    safe_gate: bool = False,
    lower_bound: float | None = None,
    disable_recompute: bool = False,
    return_intermediate_states: bool = False,
    transpose_state_layout: bool = False,
    **kwargs: Any,
):
    """Chunkwise gdn2 forward with autograd (reference ``chunk_gdn2.py:1268-1434``).

    Shapes: ``q, k, g, b [B,T,H,K]``, ``v, w [B,T,H,V]``, ``initial_state [N,H,K,V]`` float32
    (``[N,H,V,K]`` with ``transpose_state_layout``). The chunk size is 64, as in the reference
    accelerated op.

    Returns ``(o, final_state)``. Under ``torch.inference_mode`` with
    ``return_intermediate_states``, it returns ``(o, final_state, h)`` instead, with ``h`` the
    per-chunk start states (``chunk_gdn2.py:1415-1421``).
    """
    _check_packed(q, initial_state, cu_seqlens)
    if initial_state is not None:
        assert initial_state.dtype == torch.float32, f"initial_state: float32 expected, got {initial_state.dtype}"
    A_log, dt_bias = None, None
    if use_gate_in_kernel:
        assert "A_log" in kwargs, "use_gate_in_kernel needs the A_log keyword argument"
        A_log, dt_bias = kwargs["A_log"], kwargs.get("dt_bias")
    if safe_gate and use_gate_in_kernel:
        if lower_bound is None:
            raise ValueError("safe_gate with the in-kernel gate needs a lower_bound value")
        if not (-5 <= lower_bound < 0):
            raise ValueError(f"lower_bound {lower_bound} lies outside [-5, 0), where the bounded gate is defined")
    if not (safe_gate and use_gate_in_kernel):
        lower_bound = None
    assert q.shape == k.shape == g.shape, (
        f"q, k and g share one [B, T, H, K] shape; got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(g.shape)}"
    )
    assert k.shape[-1] <= 256, f"key head dim {k.shape[-1]} exceeds the chunk op's limit of 256"
    assert b.shape == q.shape, f"erase gate b: expected the shape of q {tuple(q.shape)}, got {tuple(b.shape)}"
    assert w.shape == v.shape, f"write gate w: expected the shape of v {tuple(v.shape)}, got {tuple(w.shape)}"
    assert v.shape == (*q.shape[:3], v.shape[-1]), (
        f"v: expected [B, T, H, V] with the B, T, H of q {tuple(q.shape[:3])}, got {tuple(v.shape)}"
    )
    if scale is None:
        scale = k.shape[-1] ** -0.5
    _require_gpu("chunk_gdn2", q, k, v, g, b, w, initial_state)
    if return_intermediate_states and kwargs.get("bw_logits", False):
        b, w = b.sigmoid(), w.sigmoid()  # the intermediate states use the training workspace
    if return_intermediate_states:
        assert torch.is_inference_mode_enabled(), (
            "return_intermediate_states: run the call under torch.inference_mode()"
        )
        assert disable_recompute is False, (
            "return_intermediate_states cannot be combined with disable_recompute=True"
        )
        o, ht, h = chunk_gdn2_fwd(
            q, k, v, g, b, w, scale, initial_state, output_final_state, use_qk_l2norm_in_kernel,
            use_gate_in_kernel, A_log, dt_bias, lower_bound, cu_seqlens,
            transpose_state_layout=transpose_state_layout, return_intermediate_states=True,
        )
        return o.type_as(q), ht, h
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, g, b, w, A_log, dt_bias, initial_state)
    )
    if use_gate_in_kernel and needs_grad:
        # Differentiable gate in torch, then the kernels on the activated decay.
        g = gate_activation(g, A_log, dt_bias, lower_bound)
        use_gate_in_kernel, A_log, dt_bias, lower_bound = False, None, None, None
    if kwargs.get("bw_logits", False):
        # b and w given as logits (an extension of this backend): activated in the
        # kernels when no gradient is needed, by torch otherwise.
        if not needs_grad:
            o, ht = chunk_gdn2_fwd(
                q, k, v, g, b, w, scale, initial_state, output_final_state, use_qk_l2norm_in_kernel,
                use_gate_in_kernel, A_log, dt_bias, lower_bound, cu_seqlens,
                transpose_state_layout=transpose_state_layout, bw_logits=True,
            )
            return o.type_as(q), ht
        b, w = b.sigmoid(), w.sigmoid()
    return ChunkGDN2Function.apply(
        q, k, v, g, b, w, A_log, dt_bias, scale, initial_state, output_final_state,
        use_qk_l2norm_in_kernel, use_gate_in_kernel, cu_seqlens, lower_bound, transpose_state_layout,
    )


def _ptr_array(ptrs) -> int:
    """Address of a C array of three ``void *`` (unused slots NULL)."""
    arr = (ctypes.c_void_p * 3)(*(list(ptrs) + [None] * (3 - len(ptrs))))
    _ptr_array.keep.append(arr)  # alive until the call returns
    return ctypes.addressof(arr)


_ptr_array.keep = []


@torch.compiler.disable
def short_convolution(
    xs: list[torch.Tensor],
    weights: list[torch.Tensor],
    biases: list[torch.Tensor | None] | None = None,
    caches: list[torch.Tensor | None] | None = None,
    output_final_state: bool = False,
    activation: str | None = "silu",
    out_caches: list[torch.Tensor] | None = None,
) -> tuple[list[torch.Tensor], list[torch.Tensor] | None]:
    """Causal depthwise conv1d (+ SiLU) of up to three ``[B, T, D]`` tensors in one launch.

    Each tensor follows reference ``ShortConvolution.forward`` (``gdn2.py:395-430``):
    * ``weights[i]`` is the Conv1d weight ``[D, 1, W]``;
    * a single-token call convolves the cache ``[B, D, W-1]`` followed by the new token;
    * with ``output_final_state`` the new cache holds the last ``min(T, W-1)`` inputs (``W-1`` when ``T == 1``).

    Inputs may be column ranges of a wider ``[B, T, N]`` tensor (unit channel stride, rows
    ``stride(1)`` apart): they are read in place, with no copy.

    ``out_caches`` (an extension of this backend; single-token calls only): contiguous
    ``[B, D, W-1]`` tensors that receive the new caches, possibly the input caches
    themselves (each cache entry is read before it is overwritten, by the same lane).

    Returns ``(ys, new_caches)``. Inference only: there is no backward.
    """
    name = "short_convolution"
    n = len(xs)
    if not 1 <= n <= 3 or len(weights) != n:
        raise ValueError(f"{name}: 1 to 3 tensors with one weight each")
    _require_gpu(name, *xs)
    B, T = xs[0].shape[:2]
    dt = xs[0].dtype
    W = int(weights[0].shape[-1])
    if activation not in (None, "silu"):
        raise NotImplementedError(f"{name}: activation {activation!r}")
    for x in xs:
        if x.dim() != 3 or tuple(x.shape[:2]) != (B, T):
            raise ValueError(f"{name}: inputs must share [B, T, D]; got {tuple(x.shape)}")

    def row_stride(x: torch.Tensor) -> int | None:
        """Element distance of consecutive (b, t) rows, or None if rows are not evenly spaced."""
        if x.dtype != dt or x.stride(2) != 1:
            return None
        if T > 1:
            ok = x.stride(1) >= x.shape[2] and (B <= 1 or x.stride(0) == T * x.stride(1))
            return x.stride(1) if ok else None
        if B > 1:
            return x.stride(0) if x.stride(0) >= x.shape[2] else None
        return x.shape[2]

    xs = [x if row_stride(x) is not None else x.to(dt).contiguous() for x in xs]
    ldx = (ctypes.c_int64 * 3)(*([row_stride(x) for x in xs] + [0] * (3 - n)))
    dims = [x.shape[2] for x in xs]
    ws = [w.detach().reshape(d, W).to(dt).contiguous() for w, d in zip(weights, dims)]
    bs = None
    if biases is not None and any(b_ is not None for b_ in biases):
        bs = [None if b_ is None else b_.detach().to(dt).contiguous() for b_ in biases]
    cs = None
    if T == 1 and caches is not None and any(c is not None for c in caches):
        cs = [None if c is None else c.to(dt).contiguous() for c in caches]
        for c, d in zip(cs, dims):
            if c is not None and tuple(c.shape) != (B, d, W - 1):
                raise ValueError(f"{name}: cache must be {(B, d, W - 1)}; got {tuple(c.shape)}")
    keep = W - 1 if T == 1 else min(T, W - 1)
    if out_caches is not None:
        if T != 1 or not output_final_state or len(out_caches) != n:
            raise ValueError(f"{name}: out_caches needs a single-token call with output_final_state")
        for c, d in zip(out_caches, dims):
            if tuple(c.shape) != (B, d, W - 1) or c.dtype != dt or not c.is_contiguous():
                raise ValueError(f"{name}: out_caches must be contiguous {(B, d, W - 1)} {dt} tensors")
        new = list(out_caches)
    else:
        new = [torch.empty(B, d, keep, dtype=dt, device=x.device) for x, d in zip(xs, dims)] \
            if output_final_state else None
    ys = [torch.empty_like(x) for x in xs]
    dims_arr = (ctypes.c_int * 3)(*(dims + [dims[0]] * (3 - n)))
    lib = nat.load()
    st = lib.gdn2_short_conv_fwd_ex(
        n, _ptr_array([nat.ptr(x) for x in xs]), ctypes.addressof(ldx), _ptr_array([nat.ptr(w) for w in ws]),
        None if bs is None else _ptr_array([nat.ptr(b_) for b_ in bs]),
        None if cs is None else _ptr_array([nat.ptr(c) for c in cs]),
        None if new is None else _ptr_array([nat.ptr(c) for c in new]),
        _ptr_array([nat.ptr(y) for y in ys]), ctypes.addressof(dims_arr),
        nat.dtype_code(dt), B, T, W, int(activation == "silu"), nat.stream_handle(xs[0].device),
    )
    _ptr_array.keep.clear()
    nat.check(st, name)
    return ys, new


@torch.compiler.disable
def chunk_gdn2_gated_norm(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    gate: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float = 1e-5,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    lower_bound: float | None = None,
    cu_seqlens: torch.LongTensor | None = None,
    bw_logits: bool = False,
):
    """``chunk_gdn2`` followed by the module's gated output norm, in one pass over the output.

    The norm (``RMSNormGated``, reference ``gdn2.py:433-452``) runs in the scan's output stage,
    with the roundings of :func:`gated_rmsnorm`: the result equals
    ``gated_rmsnorm(chunk_gdn2(...)[0], gate, norm_weight, eps)`` bit for bit.

    * ``gate``: ``[B, T, H, V]`` or ``[B, T, H * V]`` in the inputs' dtype; the token rows may be
      a column range of a wider tensor (unit channel stride, one row stride).
    * ``norm_weight``: ``[V]`` in the inputs' dtype.

    Inference only (no autograd); bfloat16 inputs with ``V`` in {16, 32, 64}, where one scan
    workgroup owns a whole value row. Returns ``(o, final_state)``.
    """
    name = "chunk_gdn2_gated_norm"
    _require_gpu(name, q, k, v, g, b, w, gate, norm_weight, initial_state)
    _check_shapes(name, q, k, v, g, b, w, same_heads=True)
    _check_packed(q, initial_state, cu_seqlens)
    B, T, H, K = q.shape
    V = v.shape[-1]
    dt = q.dtype
    if dt != torch.bfloat16 or V not in (16, 32, 64):
        raise NotImplementedError(f"{name}: bfloat16 inputs with a value head dim of 16, 32 or 64 "
                                  f"(got {dt}, {V})")
    if norm_weight.numel() != V or norm_weight.dtype != dt:
        raise ValueError(f"{name}: norm_weight must hold {V} {dt} values")
    gt = gate.reshape(B, T, H * V) if gate.dim() == 4 and gate.stride(-2) == V else gate
    if (gt.dim() != 3 or gt.dtype != dt or tuple(gt.shape) != (B, T, H * V) or gt.stride(-1) != 1
            or (B > 1 and gt.stride(0) != T * gt.stride(1))):
        raise ValueError(f"{name}: gate must be [B, T, H * V] {dt} token rows with unit channel stride; "
                         f"got {tuple(gate.shape)} {gate.dtype} strides {gate.stride()}")
    ld_gate = gt.stride(1) if T > 1 else max(gt.stride(1), H * V)
    if scale is None:
        scale = K ** -0.5
    q, k, v, b, w = (_io(x, dt) for x in (q, k, v, b, w))
    g = _io(g, g.dtype if g.dtype in (torch.float32, dt) else torch.float32)
    cu_dev, cu_host = _cu(cu_seqlens, q.device, T)
    N = B if cu_seqlens is None else cu_host.numel() - 1
    h0 = None if initial_state is None else initial_state.float().contiguous()
    if h0 is not None and tuple(h0.shape) != (N, H, K, V):
        raise ValueError(f"{name}: initial_state must be {(N, H, K, V)}, got {tuple(h0.shape)}")
    ht = torch.empty(N, H, K, V, dtype=torch.float32, device=q.device) if output_final_state else None
    o = torch.empty_like(v)
    lib = nat.load()
    cu_host_p = None if cu_host is None else cu_host.data_ptr()
    ws_bytes = lib.gdn2_chunk_fwd_workspace_size(B, T, H, K, V, nat.dtype_code(dt), cu_host_p, N)
    if ws_bytes == 0 and B * T > 0 and K > 128:
        raise NotImplementedError(f"{name}: key head dim {K} beyond the chunk kernels' 256")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    a_log, dtb = _gate_tensors(use_gate_in_kernel, A_log, dt_bias, H, K)
    flags = _flags(use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound)
    if bw_logits:
        flags |= nat.FLAG_SIGMOID_BW
    wn = norm_weight.detach().contiguous()
    st = lib.gdn2_chunk_fwd_gated_norm(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(g), nat.ptr(b), nat.ptr(w),
        nat.dtype_code(dt), nat.dtype_code(g.dtype), nat.ptr(o), nat.ptr(gt), ld_gate, nat.ptr(wn),
        float(eps), nat.ptr(h0), nat.ptr(ht), nat.ptr(a_log), nat.ptr(dtb),
        float(lower_bound) if lower_bound is not None else 0.0,
        nat.ptr(cu_dev), cu_host_p, N, B, T, H, K, V, float(scale), flags,
        ws.data_ptr(), ws.numel(), nat.stream_handle(q.device),
    )
    nat.check(st, name)
    return o, ht


def _raw_rows(name: str, nm: str, x: torch.Tensor, B: int, T: int, width: int, dt: torch.dtype) -> int:
    """Token row stride of a ``[B, T, width]`` (or ``[B, T, H, D]``) tensor read in place: unit
    channel stride, one row stride, 16-byte aligned rows."""
    if x.dim() == 4:
        if x.stride(-1) != 1 or x.stride(-2) != x.shape[-1]:
            raise ValueError(f"{name}: {nm} heads must be contiguous within a token row")
        x = x.flatten(-2)
    if (x.dim() != 3 or x.dtype != dt or tuple(x.shape) != (B, T, width) or x.stride(-1) != 1
            or (B > 1 and x.stride(0) != T * x.stride(1))):
        raise ValueError(f"{name}: {nm} must be [B, T, {width}] {dt} token rows with unit channel stride; "
                         f"got {tuple(x.shape)} {x.dtype} strides {x.stride()}")
    ld = x.stride(1) if T > 1 else max(x.stride(1), width)
    if ld % 8 or x.data_ptr() % 16:
        raise ValueError(f"{name}: {nm} rows must start on 16-byte boundaries (row stride {ld})")
    return ld


@torch.compiler.disable
def chunk_gdn2_conv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    conv_weights: list[torch.Tensor],
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    *,
    num_heads: int,
    activation: str | None = "silu",
    gate: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-5,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    lower_bound: float | None = None,
    cu_seqlens: torch.LongTensor | None = None,
    bw_logits: bool = False,
):
    """``chunk_gdn2`` on the raw q / k / v projections, with the module's short convolutions
    (reference ``ShortConvolution``, ``gdn2.py:395-430``: causal depthwise conv1d of width 4, no
    bias, then ``activation``) applied inside the chunk kernels.

    * ``q``, ``k``: ``[B, T, H * K]`` raw projections, ``v``: ``[B, T, H * V]``; the token rows may
      be column ranges of a wider tensor (one row stride, unit channel stride, 16-byte aligned).
    * ``conv_weights``: the three Conv1d weights ``[D, 1, 4]`` of q, k, v.
    * ``g``, ``b``, ``w``: as for :func:`chunk_gdn2` (``[B, T, H, K]`` / ``[B, T, H, V]``).
    * ``gate`` / ``norm_weight``: optional; applies the gated output norm as
      :func:`chunk_gdn2_gated_norm` does.

    Rows before a sequence's first token are zero (the prefill padding of the reference, per
    ``cu_seqlens`` sequence). Each convolution output is rounded to the input dtype before and
    after the SiLU, as in :func:`short_convolution`, so without ``cu_seqlens`` the result equals
    ``short_convolution`` followed by ``chunk_gdn2`` (or ``chunk_gdn2_gated_norm``) bit for bit.
    The new conv caches are the last three raw rows, which the caller slices itself.

    Inference only; bfloat16 inputs, ``K`` in {32, 64, 128}, ``V`` a multiple of 16 (with a gate:
    16, 32 or 64). Returns ``(o, final_state)`` with ``o`` ``[B, T, H, V]``.
    """
    name = "chunk_gdn2_conv"
    _require_gpu(name, q, k, v, g, b, w, gate, norm_weight, initial_state)
    if activation not in (None, "silu"):
        raise NotImplementedError(f"{name}: activation {activation!r}; the kernels apply SiLU or nothing")
    B, T = q.shape[0], q.shape[1]
    H = int(num_heads)
    if g.dim() != 4 or tuple(g.shape[:3]) != (B, T, H):
        raise ValueError(f"{name}: g must be [B, T, {H}, K]; got {tuple(g.shape)}")
    K = g.shape[-1]
    if w.dim() != 4 or tuple(w.shape[:3]) != (B, T, H):
        raise ValueError(f"{name}: w must be [B, T, {H}, V]; got {tuple(w.shape)}")
    V = w.shape[-1]
    if tuple(b.shape) != (B, T, H, K):
        raise ValueError(f"{name}: b must be {(B, T, H, K)}; got {tuple(b.shape)}")
    _check_packed(q, initial_state, cu_seqlens)
    dt = q.dtype
    if dt != torch.bfloat16 or K not in (32, 64, 128) or V % 16:
        raise NotImplementedError(f"{name}: bfloat16 inputs with K in (32, 64, 128) and V a multiple of 16 "
                                  f"(got {dt}, K={K}, V={V})")
    if gate is not None and V not in (16, 32, 64):
        raise NotImplementedError(f"{name}: the fused output norm needs V in (16, 32, 64), got {V}")
    ldq = _raw_rows(name, "q", q, B, T, H * K, dt)
    ldk = _raw_rows(name, "k", k, B, T, H * K, dt)
    ldv = _raw_rows(name, "v", v, B, T, H * V, dt)
    if len(conv_weights) != 3:
        raise ValueError(f"{name}: conv_weights must hold the q, k and v weights")
    taps = []
    for nm, wt, d in zip("qkv", conv_weights, (H * K, H * K, H * V)):
        if wt.numel() != d * 4:
            raise NotImplementedError(f"{name}: {nm} convolution must be [{d}, 1, 4] (width 4); "
                                      f"got {tuple(wt.shape)}")
        taps.append(_io(wt.detach().reshape(d, 4), dt))
    ld_gate, gt, wn = 0, None, None
    if gate is not None:
        if norm_weight is None or norm_weight.numel() != V or norm_weight.dtype != dt:
            raise ValueError(f"{name}: norm_weight must hold {V} {dt} values")
        gt = gate.reshape(B, T, H * V) if gate.dim() == 4 and gate.stride(-2) == V else gate
        if (gt.dim() != 3 or gt.dtype != dt or tuple(gt.shape) != (B, T, H * V) or gt.stride(-1) != 1
                or (B > 1 and gt.stride(0) != T * gt.stride(1))):
            raise ValueError(f"{name}: gate must be [B, T, H * V] {dt} token rows with unit channel "
                             f"stride; got {tuple(gate.shape)} {gate.dtype} strides {gate.stride()}")
        ld_gate = gt.stride(1) if T > 1 else max(gt.stride(1), H * V)
        wn = norm_weight.detach().contiguous()
    if scale is None:
        scale = K ** -0.5
    b, w = (_io(x, dt) for x in (b, w))
    g = _io(g, g.dtype if g.dtype in (torch.float32, dt) else torch.float32)
    cu_dev, cu_host = _cu(cu_seqlens, q.device, T)
    N = B if cu_seqlens is None else cu_host.numel() - 1
    h0 = None if initial_state is None else initial_state.float().contiguous()
    if h0 is not None and tuple(h0.shape) != (N, H, K, V):
        raise ValueError(f"{name}: initial_state must be {(N, H, K, V)}, got {tuple(h0.shape)}")
    ht = torch.empty(N, H, K, V, dtype=torch.float32, device=q.device) if output_final_state else None
    o = torch.empty(B, T, H, V, dtype=dt, device=q.device)
    lib = nat.load()
    cu_host_p = None if cu_host is None else cu_host.data_ptr()
    ws_bytes = lib.gdn2_chunk_fwd_workspace_size(B, T, H, K, V, nat.dtype_code(dt), cu_host_p, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    a_log, dtb = _gate_tensors(use_gate_in_kernel, A_log, dt_bias, H, K)
    flags = _flags(use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound)
    if bw_logits:
        flags |= nat.FLAG_SIGMOID_BW
    st = lib.gdn2_chunk_fwd_conv(
        nat.ptr(q), ldq, nat.ptr(k), ldk, nat.ptr(v), ldv, nat.ptr(taps[0]), nat.ptr(taps[1]),
        nat.ptr(taps[2]), 4, int(activation == "silu"), nat.ptr(g), nat.ptr(b), nat.ptr(w),
        nat.dtype_code(dt), nat.dtype_code(g.dtype), nat.ptr(o), nat.ptr(gt), ld_gate, nat.ptr(wn),
        float(eps), nat.ptr(h0), nat.ptr(ht), nat.ptr(a_log), nat.ptr(dtb),
        float(lower_bound) if lower_bound is not None else 0.0,
        nat.ptr(cu_dev), cu_host_p, N, B, T, H, K, V, float(scale), flags,
        ws.data_ptr(), ws.numel(), nat.stream_handle(q.device),
    )
    nat.check(st, name)
    return o, ht


@torch.compiler.disable
def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * weight * silu(z)`` over the last axis.

    This is reference ``RMSNormGated.forward`` (``gdn2.py:433-452``), rounded to the input dtype after every op as the reference is.

    Output dtype:
    * the input dtype;
    * float32 when ``weight`` is float32 and ``x`` is not (torch's promotion).

    Inference only: there is no backward.
    """
    name = "gated_rmsnorm"
    _require_gpu(name, x, z, weight)
    if z.shape != x.shape or weight.numel() != x.shape[-1]:
        raise ValueError(f"{name}: x, z must match and weight must have {x.shape[-1]} elements")
    dt = x.dtype
    N = x.shape[-1]
    xc = x.contiguous()
    zc = z.to(dt).contiguous()
    wd = weight.detach()
    wdt = torch.float32 if (wd.dtype == torch.float32 and dt != torch.float32) else dt
    wc = wd.to(wdt).contiguous()
    out = torch.empty(x.shape, dtype=wdt, device=x.device)
    lib = nat.load()
    st = lib.gdn2_gated_rmsnorm_fwd(
        nat.ptr(xc), nat.ptr(zc), nat.ptr(wc), nat.dtype_code(wdt), nat.ptr(out), nat.dtype_code(dt),
        xc.numel() // N, N, float(eps), nat.stream_handle(x.device),
    )
    nat.check(st, name)
    return out


class ShortConvFunction(torch.autograd.Function):
    """Prefill ``ShortConvolution`` (no cache) with the HIP forward and backward.

    Forward: :func:`short_convolution` (``gdn2.py:395-430`` with the reference's rounding).
    Backward: ``gdn2_short_conv_bwd`` -- the gradients torch's autograd gives through
    ``F.conv1d`` and ``F.silu``, in fp32 with deterministic sums.
    """

    @staticmethod
    def forward(ctx, x, weight, bias, silu: bool):
        (y,), _ = short_convolution([x], [weight], [bias], None, False, "silu" if silu else None)
        ctx.save_for_backward(x, weight, bias)
        ctx.silu = silu
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, bias = ctx.saved_tensors
        name = "short_convolution backward"
        B, T, D = x.shape
        W = int(weight.shape[-1])
        dt = x.dtype
        xc = x if (x.stride(2) == 1 and (B <= 1 or x.stride(0) == T * x.stride(1)) and x.stride(1) >= D) \
            else x.contiguous()
        ld = xc.stride(1) if T > 1 else (xc.stride(0) if B > 1 else D)
        dyc = dy.to(dt).contiguous()
        wc = weight.detach().reshape(D, W).to(dt).contiguous()
        bc = None if bias is None else bias.detach().to(dt).contiguous()
        dx = torch.empty(B, T, D, dtype=dt, device=x.device)
        dw = torch.empty(D, W, dtype=dt, device=x.device)
        db = None if bias is None else torch.empty(D, dtype=dt, device=x.device)
        lib = nat.load()
        wsb = lib.gdn2_short_conv_bwd_workspace_size(B, T, D, W)
        ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=x.device)
        st = lib.gdn2_short_conv_bwd(nat.ptr(xc), ld, nat.ptr(wc), nat.ptr(bc), nat.ptr(dyc), nat.ptr(dx),
                                     nat.ptr(dw), nat.ptr(db), nat.dtype_code(dt), B, T, D, W, int(ctx.silu),
                                     ws.data_ptr(), ws.numel(), nat.stream_handle(x.device))
        nat.check(st, name)
        dwo = dw.reshape(weight.shape).to(weight.dtype)
        dbo = None if db is None else db.to(bias.dtype)
        return dx, dwo, dbo, None


@torch.compiler.disable
def short_conv_autograd(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                        activation: str | None = "silu") -> torch.Tensor:
    """Differentiable prefill short convolution (no cache) on the HIP kernels; ``[B, T, D]`` in
    and out, ``weight`` the Conv1d weight ``[D, 1, W]`` (W <= 8)."""
    _require_gpu("short_conv_autograd", x)
    if activation not in (None, "silu"):
        raise NotImplementedError(f"short_conv_autograd: activation {activation!r}")
    return ShortConvFunction.apply(x, weight, bias, activation == "silu")


class GatedRMSNormFunction(torch.autograd.Function):
    """``RMSNormGated`` with the HIP forward (:func:`gated_rmsnorm`, the reference's rounding)
    and backward (``gdn2_gated_rmsnorm_bwd``: dx, dz, dweight in fp32, deterministic)."""

    @staticmethod
    def forward(ctx, x, z, weight, eps: float):
        out = gated_rmsnorm(x, z, weight, eps)
        ctx.save_for_backward(x, z, weight)
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, dout):
        x, z, weight = ctx.saved_tensors
        name = "gated_rmsnorm backward"
        dt = x.dtype
        N = x.shape[-1]
        xc, zc = x.contiguous(), z.to(dt).contiguous()
        wdt = torch.float32 if weight.dtype == torch.float32 else dt
        wc = weight.detach().to(wdt).contiguous()
        dyc = dout.to(dt).contiguous()
        rows = xc.numel() // N
        dx, dz = torch.empty_like(xc), torch.empty_like(zc)
        dw = torch.empty(N, dtype=wdt, device=x.device)
        lib = nat.load()
        wsb = lib.gdn2_gated_rmsnorm_bwd_workspace_size(rows, N)
        ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=x.device)
        st = lib.gdn2_gated_rmsnorm_bwd(nat.ptr(xc), nat.ptr(zc), nat.ptr(wc), nat.dtype_code(wdt), nat.ptr(dyc),
                                        nat.ptr(dx), nat.ptr(dz), nat.ptr(dw), nat.dtype_code(dt), rows, N,
                                        float(ctx.eps), ws.data_ptr(), ws.numel(), nat.stream_handle(x.device))
        nat.check(st, name)
        return dx, dz.to(z.dtype), dw.to(weight.dtype), None


@torch.compiler.disable
def gated_rmsnorm_autograd(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor,
                           eps: float = 1e-5) -> torch.Tensor:
    """Differentiable gated RMS norm on the HIP kernels (rows of up to 256 values)."""
    _require_gpu("gated_rmsnorm_autograd", x, z, weight)
    if x.shape[-1] > 256:
        raise NotImplementedError("gated_rmsnorm_autograd: rows of up to 256 values")
    return GatedRMSNormFunction.apply(x, z, weight, eps)


@torch.compiler.disable
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``weight * (x * rsqrt(mean(x^2) + eps))`` over the last axis (N <= 2048).

    This is reference ``RMSNorm.forward`` (``models/normalization.py:40-51``), the decoder
    hosts' norm, rounded to the input dtype after every op as the reference is.  It runs
    on the gated norm's entry point with the gate left out.

    Output dtype: as for ``gated_rmsnorm``.  Inference only: there is no backward.
    """
    name = "rms_norm"
    _require_gpu(name, x, weight)
    if weight.numel() != x.shape[-1]:
        raise ValueError(f"{name}: weight must have {x.shape[-1]} elements")
    dt = x.dtype
    N = x.shape[-1]
    xc = x.contiguous()
    wd = weight.detach()
    wdt = torch.float32 if (wd.dtype == torch.float32 and dt != torch.float32) else dt
    wc = wd.to(wdt).contiguous()
    out = torch.empty(x.shape, dtype=wdt, device=x.device)
    lib = nat.load()
    st = lib.gdn2_gated_rmsnorm_fwd(
        nat.ptr(xc), None, nat.ptr(wc), nat.dtype_code(wdt), nat.ptr(out), nat.dtype_code(dt),
        xc.numel() // N, N, float(eps), nat.stream_handle(x.device),
    )
    nat.check(st, name)
    return out


@torch.compiler.disable
def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float = 1e-5) -> tuple[torch.Tensor, torch.Tensor]:
    """``s = x + residual`` and ``rms_norm(s, weight, eps)`` in one pass; returns ``(s, norm)``.

    The decoder hosts' ``x = x + h`` followed by the next ``RMSNorm`` (reference
    ``gdn2_gpt/model.py:240-248``, ``models/normalization.py:40-51``), equal to the two
    separate ops bit for bit.  Rows of ``N`` values with ``N`` times the element size a
    power of two between 64 and 4096 bytes; other shapes raise ``NotImplementedError``
    (``add_rms_norm_supported`` tells them apart).  Inference only.
    """
    name = "add_rms_norm"
    _require_gpu(name, x, residual, weight)
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError(f"{name}: residual must match x in shape and dtype")
    if weight.numel() != x.shape[-1]:
        raise ValueError(f"{name}: weight must have {x.shape[-1]} elements")
    dt = x.dtype
    N = x.shape[-1]
    xc, rc = x.contiguous(), residual.contiguous()
    wd = weight.detach()
    wdt = torch.float32 if (wd.dtype == torch.float32 and dt != torch.float32) else dt
    wc = wd.to(wdt).contiguous()
    s = torch.empty_like(xc)
    out = torch.empty(x.shape, dtype=wdt, device=x.device)
    lib = nat.load()
    st = lib.gdn2_add_rms_norm_fwd(
        nat.ptr(xc), nat.ptr(rc), nat.ptr(s), nat.ptr(wc), nat.dtype_code(wdt), nat.ptr(out),
        nat.dtype_code(dt), xc.numel() // N, N, float(eps), nat.stream_handle(x.device),
    )
    if st == nat.ERR_UNSUPPORTED:
        raise NotImplementedError(f"{name}: rows of {N} {dt} values are not supported")
    nat.check(st, name)
    return s, out


def add_rms_norm_supported(x: torch.Tensor) -> bool:
    """Whether ``add_rms_norm`` takes rows of ``x``'s width and dtype."""
    nbytes = x.shape[-1] * x.element_size()
    return nbytes % 16 == 0 and 4 <= nbytes // 16 <= 256 and (nbytes // 16) & (nbytes // 16 - 1) == 0


@torch.compiler.disable
def silu_mul(ab: torch.Tensor) -> torch.Tensor:
    """``F.silu(a) * b`` for ``a, b = ab.chunk(2, dim=-1)``: SwiGLU's gated product
    (reference ``gdn2_gpt/model.py:74-77``) on the output of one fused w1 / w2
    projection, with torch's rounding to the io dtype after each op.  The last axis of
    ``ab`` has unit stride; the other axes may be strided as rows.  Inference only."""
    name = "silu_mul"
    _require_gpu(name, ab)
    dt = ab.dtype
    if ab.shape[-1] % 2:
        raise ValueError(f"{name}: the last axis must have an even length")
    H = ab.shape[-1] // 2
    a2 = ab.reshape(-1, 2 * H) if ab.dim() != 2 else ab
    if a2.stride(-1) != 1:
        a2 = a2.contiguous()
    ld = a2.stride(0) if a2.shape[0] > 1 else 2 * H  # a single row's stride is arbitrary
    out = torch.empty(ab.shape[:-1] + (H,), dtype=dt, device=ab.device)
    lib = nat.load()
    st = lib.gdn2_silu_mul_fwd(
        nat.ptr(a2), ld, nat.ptr(out), nat.dtype_code(dt), a2.shape[0], H,
        nat.stream_handle(ab.device),
    )
    if st == nat.ERR_UNSUPPORTED:
        raise NotImplementedError(f"{name}: {H} {dt} columns are not supported")
    nat.check(st, name)
    return out


_SKINNY_NP = (1, 2, 4, 6, 8)
# Wider outputs (an LM head) stay on torch's GEMM, which reads a weight of that size
# faster (measured at the config-3 decode step; the few-row kernel wins below).
_SKINNY_MAX_N = 16384


@torch.compiler.disable
def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)``, on the HIP few-row kernel when ``x`` has at most 8
    rows (a decode step's batch; at most 4 beyond K = 2048), at most 16384 output
    columns, 16-bit inputs and ``K / 512`` in {1, 2, 4, 6, 8};
    other calls, and calls through which a gradient flows, are torch's GEMM.

    The kernel reads each row of ``weight`` once with every request in flight before any
    arithmetic (the product is a read of the weight at this size) and accumulates in
    fp32, rounding once as torch does; its summation order differs from torch's GEMM,
    so results agree to rounding, not bit for bit.
    """
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    if (not x.is_cuda or weight.shape[0] > _SKINNY_MAX_N or x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype
            or (bias is not None and bias.dtype != x.dtype) or not 1 <= M <= 8 or K % 512
            or K // 512 not in _SKINNY_NP or (M > 4 and K > 2048) or weight.dim() != 2 or weight.stride(1) != 1
            or (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, weight, bias)))):
        return F.linear(x, weight, bias)
    x2 = x.reshape(M, K)
    if x2.stride(1) != 1 or (M > 1 and x2.stride(0) % 8):
        x2 = x2.contiguous()
    N = weight.shape[0]
    b = None if bias is None else bias.contiguous()
    y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
    lib = nat.load()
    st = lib.gdn2_skinny_linear(
        nat.ptr(x2), x2.stride(0) if M > 1 else K, nat.ptr(weight), weight.stride(0), nat.ptr(b),
        nat.ptr(y), N, nat.dtype_code(x.dtype), M, N, K, nat.stream_handle(x.device),
    )
    if st == nat.ERR_UNSUPPORTED:  # alignment: torch's GEMM
        return F.linear(x, weight, bias)
    nat.check(st, "linear")
    return y


@torch.compiler.disable
def linear_addnorm(x: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                   weight: torch.Tensor, bias: torch.Tensor | None = None,
                   swiglu: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """``s, n = add_rms_norm(x, residual, norm_weight, eps); return linear(n, weight, bias), s``
    in one launch on decode-sized rows (at most 4, K in {512, 1024, 2048}, 16-bit, the
    norm weight in the io dtype): the normalised rows are formed while the few-row
    kernel stages its input, bit for bit as the two ops.  With ``swiglu`` (``weight`` the
    stacked [w1; w2]) the first output is ``silu_mul`` of the product, formed in the
    kernel's epilogue.  Other shapes run the separate ops."""
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = weight.shape[0]
    if (x.is_cuda and (not swiglu or N % 2 == 0) and x.dtype in (torch.bfloat16, torch.float16) and 1 <= M <= 4 and K in (512, 1024, 2048)
            and residual.shape == x.shape and residual.dtype == x.dtype and norm_weight.dtype == x.dtype
            and norm_weight.numel() == K and weight.dtype == x.dtype and weight.dim() == 2 and weight.shape[1] == K
            and weight.stride(1) == 1 and N <= _SKINNY_MAX_N and (bias is None or bias.dtype == x.dtype)
            and not (torch.is_grad_enabled()
                     and any(t is not None and t.requires_grad for t in (x, residual, norm_weight, weight, bias)))):
        xc, rc = x.reshape(M, K).contiguous(), residual.reshape(M, K).contiguous()
        nwc = norm_weight.detach().contiguous()
        s = torch.empty_like(x)
        NO = N // 2 if swiglu else N
        y = torch.empty(x.shape[:-1] + (NO,), dtype=x.dtype, device=x.device)
        b = None if bias is None else bias.contiguous()
        lib = nat.load()
        fn = lib.gdn2_skinny_linear_addnorm_swiglu if swiglu else lib.gdn2_skinny_linear_addnorm
        st = fn(
            nat.ptr(xc), K, nat.ptr(rc), K, nat.ptr(s), K, nat.ptr(nwc), float(eps), nat.ptr(weight),
            weight.stride(0), nat.ptr(b), nat.ptr(y), NO, nat.dtype_code(x.dtype), M, N, K,
            nat.stream_handle(x.device),
        )
        if st != nat.ERR_UNSUPPORTED:
            nat.check(st, "linear_addnorm")
            return y, s
    s, n = add_rms_norm(x, residual, norm_weight, eps)
    y = linear(n, weight, bias)
    if not swiglu:
        return y, s
    try:
        return silu_mul(y), s
    except NotImplementedError:  # widths silu_mul's 16-byte pieces do not cover
        a, b = y.chunk(2, dim=-1)
        return F.silu(a) * b, s


@torch.compiler.disable
def linear_pair(x0: torch.Tensor, w0: torch.Tensor, b0: torch.Tensor | None, x1: torch.Tensor,
                w1: torch.Tensor, b1: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """``(F.linear(x0, w0, b0), F.linear(x1, w1, b1))`` in one HIP launch when both have
    the same few rows (at most min(8, K / 8)) and a small inner dimension K in {32, 64,
    128, 256}: the module's second-stage gate projections (``f_proj[1]``, ``g_proj[1]``)
    of a decode step.  Other calls, and calls with gradients, are torch's GEMMs.  fp32
    sums rounded once (torch's GEMM agrees to rounding)."""
    K = x0.shape[-1]
    M = x0.numel() // K if K else 0
    ok = (x0.is_cuda and x0.dtype in (torch.bfloat16, torch.float16) and K in (32, 64, 128, 256)
          and 1 <= M <= min(8, K // 8) and x1.shape[-1] == K and x1.numel() == M * K
          and all(t.dtype == x0.dtype for t in (x1, w0, w1)) and all(b is None or b.dtype == x0.dtype for b in (b0, b1))
          and w0.shape[1] == K and w1.shape[1] == K
          and not (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x0, x1, w0, w1, b0, b1))))
    if not ok:
        return F.linear(x0, w0, b0), F.linear(x1, w1, b1)
    xs = []
    for x in (x0, x1):
        x2 = x.reshape(M, K)
        if x2.stride(1) != 1 or (M > 1 and x2.stride(0) % 8):
            x2 = x2.contiguous()
        xs.append(x2)
    wc = [w.contiguous() for w in (w0, w1)]
    bc = [None if b is None else b.contiguous() for b in (b0, b1)]
    ys = [torch.empty(x.shape[:-1] + (w.shape[0],), dtype=x.dtype, device=x.device) for x, w in ((x0, w0), (x1, w1))]
    lib = nat.load()
    st = lib.gdn2_small_linear_pair(
        nat.ptr(xs[0]), xs[0].stride(0) if M > 1 else K, nat.ptr(wc[0]), nat.ptr(bc[0]), nat.ptr(ys[0]), w0.shape[0],
        w0.shape[0], nat.ptr(xs[1]), xs[1].stride(0) if M > 1 else K, nat.ptr(wc[1]), nat.ptr(bc[1]), nat.ptr(ys[1]),
        w1.shape[0], w1.shape[0], nat.dtype_code(x0.dtype), M, K, nat.stream_handle(x0.device),
    )
    if st == nat.ERR_UNSUPPORTED:  # alignment: torch's GEMMs
        return F.linear(x0, w0, b0), F.linear(x1, w1, b1)
    nat.check(st, "linear_pair")
    return ys[0], ys[1]


@torch.compiler.disable
def argmax_rows(x: torch.Tensor, out: torch.Tensor | None = None, split: bool = True) -> torch.Tensor:
    """``x.argmax(-1, keepdim=True)`` of a 2-D tensor of logits on the HIP kernels (the
    first index of the maximum, NaN counting as the maximum, as torch's argmax), written
    to ``out`` (int64 ``[rows, 1]``, any row stride) when given.  Rows longer than 1024
    16-byte pieces are split over several workgroups and merged by a second launch
    (workspace allocated here); ``split=False`` keeps one workgroup per row, one launch.
    Rows whose layout the kernel does not take use torch's argmax."""
    if x.dim() != 2:
        raise ValueError("argmax_rows: x must be 2-D [rows, n]")
    rows, n = x.shape
    if out is None:
        out = torch.empty(rows, 1, dtype=torch.int64, device=x.device)
    elif out.dtype != torch.int64 or out.numel() != rows:
        raise ValueError("argmax_rows: out must hold one int64 per row")
    st = nat.ERR_UNSUPPORTED
    if x.is_cuda and x.dtype in (torch.bfloat16, torch.float16, torch.float32) and n > 0 and x.stride(1) == 1:
        lib = nat.load()
        dt = nat.dtype_code(x.dtype)
        ws_bytes = lib.gdn2_argmax_rows_workspace_size(rows, n, dt) if split else 0
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
        st = lib.gdn2_argmax_rows(nat.ptr(x), x.stride(0) if rows > 1 else n, dt, rows, n, nat.ptr(out),
                                  out.stride(0) if rows > 1 else 1, nat.ptr(ws), ws_bytes, nat.stream_handle(x.device))
    if st == nat.ERR_UNSUPPORTED:
        out.copy_(x.argmax(-1, keepdim=True).view(out.shape))
        return out
    nat.check(st, "argmax_rows")
    return out


def attention_decode_supported(qkv: torch.Tensor, qpk: int, head_dim: int) -> bool:
    """Whether ``attention_decode`` takes this dtype, head size and query heads per group."""
    return qkv.is_cuda and qkv.dtype in (torch.bfloat16, torch.float16) and qpk in (1, 2, 4) and head_dim in (64, 128)


@torch.compiler.disable
def attention_decode(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, input_pos: torch.Tensor,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, n_head: int) -> torch.Tensor:
    """One decode step of the hybrid host's grouped-query attention in one HIP launch:
    RoPE of the token's q heads and k, the KV-cache store at ``input_pos`` and softmax
    attention over the cache up to it (the single-token path of reference
    ``CausalSelfAttention.forward``, ``gdn2_gpt/model.py:89-173``).

    ``qkv`` ``[B, 1, G * (qpk + 2) * D]`` (the fused ``attn`` projection of one token),
    ``cos`` / ``sin`` the token's rotation ``[1, rot / 2]`` (fp32), or the whole tables
    ``[R >= L, rot / 2]`` (fp32, contiguous), whose row ``input_pos`` the kernel reads,
    ``input_pos`` ``[1]`` (device int64), caches ``[B, G, L, D]``.  Returns ``[B, n_head, D]``.  Scores and
    probabilities stay fp32 (torch's path rounds them to the io dtype), so results agree
    to that rounding.  Inference only.
    """
    name = "attention_decode"
    _require_gpu(name, qkv, cos, sin, input_pos, k_cache, v_cache)
    B, G, L, D = k_cache.shape
    qpk = n_head // G
    if qkv.numel() != B * G * (qpk + 2) * D or v_cache.shape != k_cache.shape:
        raise ValueError(f"{name}: qkv, caches and n_head do not agree")
    if input_pos.numel() != 1 or input_pos.dtype != torch.int64:
        raise ValueError(f"{name}: input_pos must be one int64 position")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.dtype == qkv.dtype == v_cache.dtype):
        raise ValueError(f"{name}: caches must be contiguous and of qkv's dtype")
    pairs = cos.shape[-1]
    if 2 * pairs > D or sin.shape != cos.shape:
        raise ValueError(f"{name}: the rotation has more than D / 2 pairs, or cos and sin differ in shape")
    qc = qkv.contiguous()
    rope_stride = 0
    if cos.dim() == 2 and cos.shape[0] > 1:
        # Whole tables: the kernel reads row input_pos (in range: positions from L on
        # leave the caches alone and read no row).
        if cos.shape[0] < L or cos.dtype != torch.float32 or sin.dtype != torch.float32 or not (
                cos.is_contiguous() and sin.is_contiguous()):
            raise ValueError(f"{name}: rotation tables must be contiguous fp32 with at least {L} rows")
        cf, sf, rope_stride = cos, sin, pairs
    else:
        cf, sf = cos.reshape(-1)[:pairs].float().contiguous(), sin.reshape(-1)[:pairs].float().contiguous()
    out = torch.empty(B, n_head, D, dtype=qkv.dtype, device=qkv.device)
    lib = nat.load()
    ws_bytes = lib.gdn2_attn_decode_workspace_size(B, G, qpk, D, L)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qkv.device) if ws_bytes else None
    st = lib.gdn2_attn_decode(
        nat.ptr(qc), nat.ptr(cf), nat.ptr(sf), pairs, rope_stride, nat.ptr(input_pos), nat.ptr(k_cache),
        nat.ptr(v_cache),
        nat.ptr(out), nat.dtype_code(qkv.dtype), B, G, qpk, D, L, float(D) ** -0.5, nat.ptr(ws), ws_bytes,
        nat.stream_handle(qkv.device),
    )
    nat.check(st, name)
    return out


def _rows2d(name: str, x: torch.Tensor, dt: torch.dtype, width: int) -> int:
    """Row stride of a [N, >= width] tensor read in place (unit channel stride)."""
    if x.dim() != 2 or x.dtype != dt or x.stride(1) != 1 or x.shape[1] < width:
        raise ValueError(f"decode_step_fused: {name} must be [N, {width}] {dt} rows with unit channel "
                         f"stride; got {tuple(x.shape)} {x.dtype} strides {x.stride()}")
    return x.stride(0) if x.shape[0] > 1 else max(x.stride(0), width)


@torch.compiler.disable
def decode_step_fused(
    x_qkv: list[torch.Tensor],
    conv_weights: list[torch.Tensor],
    conv_biases: list[torch.Tensor | None] | None,
    conv_caches: list[torch.Tensor] | None,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    initial_state: torch.Tensor | None,
    gate: torch.Tensor | None,
    norm_weight: torch.Tensor | None,
    eps: float = 1e-5,
    *,
    num_heads: int,
    head_dim: int,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    lower_bound: float | None = None,
    scale: float | None = None,
    use_qk_l2norm_in_kernel: bool = True,
    bw_logits: bool = True,
    update_cache_in_place: bool = False,
    output_final_state: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None, list[torch.Tensor] | None]:
    """One decode token per sequence through the whole mixer core (C entry ``gdn2_decode_fused``).

    Fuses, for ``num_v_heads == num_heads`` and ``K == V == head_dim`` in {64, 128}, the
    module's decode chain: ``ShortConvolution`` of q, k, v with the conv caches
    (reference ``gdn2.py:395-430``), the gate and b / w activations (``:840-866``), the
    recurrence (``fused_recurrent_gdn2.py:461-555``) and ``RMSNormGated`` of the output
    (``:433-452``).  Each stage keeps the arithmetic of its separate HIP pass.

    ``x_qkv``: the raw q, k, v projections, ``[N, H * D]`` each (column ranges of a wider
    projection output are read in place); ``g`` the decay pre-activation when ``A_log`` is
    given (else the activated decay), ``b`` / ``w`` the erase / write gates (logits when
    ``bw_logits``), ``gate`` the output gate ``g_proj(x)``, all ``[N, H * D]``.
    ``conv_weights[t]`` is the Conv1d weight ``[H * D, 1, 4]``; ``conv_caches[t]``
    ``[N, H * D, 3]`` or ``None`` (zero history).  ``initial_state`` ``[N, H, D, D]`` float32.

    Returns ``(o [N, H, D], final_state, new_conv_caches)``.  With ``update_cache_in_place``
    the conv caches and ``initial_state`` are updated where they lie and returned.
    Inference only.
    """
    name = "decode_step_fused"
    H, D = num_heads, head_dim
    HD = H * D
    _require_gpu(name, *x_qkv, g, b, w, initial_state, gate, norm_weight)
    dt = x_qkv[0].dtype
    N = x_qkv[0].shape[0]
    if len(x_qkv) != 3 or len(conv_weights) != 3:
        raise ValueError(f"{name}: q, k and v with one conv weight each")
    ld = [_rows2d(nm, x, dt, HD) for nm, x in zip(("q", "k", "v"), x_qkv)]
    g_dt = g.dtype if g.dtype in (torch.float32, dt) else None
    if g_dt is None:
        raise ValueError(f"{name}: g must be float32 or {dt}")
    ldg, ldb, ldw = _rows2d("g", g, g_dt, HD), _rows2d("b", b, dt, HD), _rows2d("w", w, dt, HD)
    ldz = 0 if gate is None else _rows2d("gate", gate, dt, HD)
    if any(x.shape[0] != N for x in (*x_qkv, g, b, w)) or (gate is not None and gate.shape[0] != N):
        raise ValueError(f"{name}: every input needs {N} rows")
    W = int(conv_weights[0].shape[-1])
    cw = [wt.detach().reshape(HD, W).to(dt).contiguous() for wt in conv_weights]
    cb = None
    if conv_biases is not None and any(x is not None for x in conv_biases):
        cb = [None if x is None else x.detach().to(dt).contiguous() for x in conv_biases]
    cin = None
    if conv_caches is not None:
        cin = list(conv_caches)
        for c in cin:
            if tuple(c.shape) != (N, HD, W - 1) or c.dtype != dt or not c.is_contiguous():
                raise ValueError(f"{name}: conv caches must be contiguous {(N, HD, W - 1)} {dt} tensors")
    if update_cache_in_place:
        if cin is None or initial_state is None:
            raise ValueError(f"{name}: update_cache_in_place needs conv caches and an initial state")
        cout, ht = cin, initial_state
    else:
        cout = [torch.empty(N, HD, W - 1, dtype=dt, device=g.device) for _ in range(3)]
        ht = torch.empty(N, H, D, D, dtype=torch.float32, device=g.device) if output_final_state else None
    for nm, st in (("initial_state", initial_state), ("final state", ht)):
        if st is not None and (st.dtype != torch.float32 or tuple(st.shape) != (N, H, D, D)
                               or st.stride()[1:] != (D * D, D, 1)):
            raise ValueError(f"{name}: {nm} must be float32 [N, H, D, D] with contiguous rows")
    nwt = None
    nw_code = nat.DTYPE_F32
    if norm_weight is not None:
        nwt = norm_weight.detach()
        nwt = nwt if nwt.dtype in (torch.float32, dt) else nwt.to(dt)
        nwt = nwt.contiguous()
        nw_code = nat.dtype_code(nwt.dtype)
    out_dt = torch.float32 if (nwt is not None and nwt.dtype == torch.float32 and dt != torch.float32) else dt
    o = torch.empty(N, H, D, dtype=out_dt, device=g.device)
    a_log, dtb = _gate_tensors(A_log is not None, A_log, dt_bias, H, D)
    flags = _flags(use_qk_l2norm_in_kernel, A_log is not None, lower_bound)
    if bw_logits:
        flags |= nat.FLAG_SIGMOID_BW
    if scale is None:
        scale = D**-0.5
    i64x3 = (ctypes.c_int64 * 3)(*ld)
    lib = nat.load()
    st = lib.gdn2_decode_fused(
        _ptr_array([nat.ptr(x) for x in x_qkv]), ctypes.addressof(i64x3),
        nat.ptr(g), ldg, nat.dtype_code(g_dt), nat.ptr(b), ldb, nat.ptr(w), ldw,
        _ptr_array([nat.ptr(x) for x in cw]), None if cb is None else _ptr_array([nat.ptr(x) for x in cb]), W,
        None if cin is None else _ptr_array([nat.ptr(x) for x in cin]), _ptr_array([nat.ptr(x) for x in cout]),
        nat.ptr(initial_state), 0 if initial_state is None else initial_state.stride(0),
        nat.ptr(ht), 0 if ht is None else ht.stride(0),
        nat.ptr(a_log), nat.ptr(dtb), float(lower_bound) if lower_bound is not None else 0.0,
        nat.ptr(gate), ldz, nat.ptr(nwt), nw_code, float(eps), nat.ptr(o),
        nat.dtype_code(dt), N, H, D, D, float(scale), flags, nat.stream_handle(g.device),
    )
    _ptr_array.keep.clear()
    nat.check(st, name)
    return o, ht, cout
