r"""CPU oracle for the gdn2 (GatedDeltaNet2) token mixer.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product package ``qwendopamine_amd`` never imports it and has no
CPU fallback.

Everything here is plain numpy in float64 (pure-Python loops only over tokens
and chunks).  Functions and the reference code they restate:

* ``l2normalize``       -- ``F.normalize(x, p=2, dim=-1, eps=1e-6)`` as used at
                           reference ``models/gdn2/gdn2.py:139-141``.
* ``recurrent_fwd``     -- ``torch_recurrent_gdn2`` (``gdn2.py:100-184``): the
                           token-by-token recurrence, the parity oracle.
                           GVA (value heads = groups x key heads) follows
                           ``fused_recurrent_gdn2.py:461-480`` (q, k indexed by
                           ``hv // groups``); varlen follows the ``cu_seqlens``
                           contract of ``fused_recurrent_gdn2.py:512-525``.
* ``chunk_fwd``         -- chunkwise WY/UT form of the same recurrence using
                           only *relative* decays ``exp(G_r - G_i) <= 1``.  It
                           is the algebra the HIP chunk kernels implement; the
                           reference's own chunk form (``gdn2.py:243-369``) uses
                           absolute decays and underflows, so it is not
                           restated.
* ``recurrent_fwd_pooled`` -- the serving options of the token-serial op
                           (``fused_recurrent_gdn2.py:215-232, 311-333``): a state
                           pool addressed through ``ssm_state_indices``
                           (continuous batching), ``num_accepted_tokens``
                           (speculative decoding), per-token state stores and
                           the transposed ``[V, K]`` state layout, around
                           ``recurrent_fwd``.
* ``recurrent_vjp``     -- reverse-mode derivative of ``recurrent_fwd``
                           (the gradients ``ChunkGDN2Function.backward`` returns,
                           ``chunk_gdn2.py:2461-2547``: dq, dk, dv, dg, db, dw,
                           dh0), including the L2-norm and scale chain rule.
* ``chunk_vjp``         -- the same derivative computed chunk by chunk (the
                           reverse state scan plus per-chunk products of the
                           reference's chunk backward, ``chunk_gdn2.py:2170-2325``:
                           recompute, dAv, dhu, wy_dqkg, intra, reverse cumsum
                           of dg), restated with relative decays.  It is the
                           algebra the HIP backward kernels implement.
* ``short_conv``        -- ``ShortConvolution.forward`` (``gdn2.py:395-430``):
                           causal depthwise conv1d + bias + SiLU with the conv
                           cache of single-token calls and the new cache.
* ``gated_rmsnorm``     -- ``RMSNormGated.forward`` (``gdn2.py:433-452``) in
                           float64 (the reference rounds each op to the input
                           dtype; the float64 value is what that rounding
                           approximates).
* ``make_inputs``       -- the seeded input recipe of BASELINE configs 0-4.

How each function is pinned (tests/test_oracle.py):
  recurrent_fwd  linear-attention closed form (b=0, w=1, g=0); single-token
                 closed form; explicit (K x K) matrix form of the update
                 ``S_t = (I - k (b*k)^T) Diag(e^g) S + k (w*v)^T`` (gdn2.py:10-11);
                 the third-party scalar gated delta rule of ``transformers``
                 (qwen3_next) for broadcast scalar gates; split/resume and
                 zero-padding invariance.
  chunk_fwd      equals recurrent_fwd for chunk sizes 1..T incl. ragged tails.
  recurrent_fwd_pooled  identity slots reduce it to recurrent_fwd; a speculative
                 step resumed from slot num_accepted-1 equals the plain
                 recurrence over the accepted tokens followed by the new ones;
                 per-token stores equal the recurrence truncated at each token;
                 the transposed layout is the swapped axes of the plain one.
  recurrent_vjp  central finite differences of recurrent_fwd in float64.
  chunk_vjp      equals recurrent_vjp for several chunk sizes incl. ragged tails.
  short_conv     per channel equals numpy's full convolution (np.convolve, with
                 the kernel flipped) truncated to T; a cached single-token call
                 equals the last row of the prefill over cache + token.
  gated_rmsnorm  equals torch.nn.functional.rms_norm (float64) times silu(z).
  make_inputs    distribution moments and l2-norms (cheap sanity only; it is a
                 recipe, not arithmetic of the reference).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "l2normalize",
    "recurrent_fwd",
    "chunk_fwd",
    "recurrent_fwd_pooled",
    "recurrent_vjp",
    "chunk_vjp",
    "make_inputs",
    "rel_l2",
    "short_conv",
    "gated_rmsnorm",
]

L2_EPS = 1e-6


def rel_l2(x, ref) -> float:
    """Relative L2 error ``||x - ref|| / ||ref||`` (the north-star parity metric)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref.ravel())
    num = np.linalg.norm((x - ref).ravel())
    if den == 0.0:
        return float(num)
    return float(num / den)


def l2normalize(x: np.ndarray, eps: float = L2_EPS) -> np.ndarray:
    """``x / max(||x||_2, eps)`` over the last axis (gdn2.py:139-141, F.normalize)."""
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    return x / np.maximum(n, eps)


def _prep(q, k, v, g, b, w, scale, use_qk_l2norm):
    q, k, v, g, b, w = (np.asarray(t, dtype=np.float64) for t in (q, k, v, g, b, w))
    if use_qk_l2norm:
        q = l2normalize(q)
        k = l2normalize(k)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    return q * scale, k, v, g, b, w


def _expand_heads(x, hv):
    """Repeat key-side heads to ``hv`` value heads (head hv uses key head hv // groups)."""
    h = x.shape[2]
    if h == hv:
        return x
    assert hv % h == 0
    return np.repeat(x, hv // h, axis=2)


def _seq_slices(B, T, cu_seqlens):
    if cu_seqlens is None:
        return [(bi, 0, T) for bi in range(B)]
    assert B == 1, "cu_seqlens requires batch size 1"
    cu = [int(c) for c in cu_seqlens]
    return [(0, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


def recurrent_fwd(
    q,
    k,
    v,
    g,
    b,
    w,
    initial_state=None,
    scale=None,
    use_qk_l2norm_in_kernel=True,
    cu_seqlens=None,
    return_states=False,
):
    r"""Token-by-token gdn2 recurrence in float64 (gdn2.py:100-184).

    Shapes: ``q, k [B,T,H,K]``; ``v, w [B,T,HV,V]``; ``g, b [B,T,HV,K]``;
    ``initial_state [N,HV,K,V]`` with ``N = B`` or ``len(cu_seqlens)-1``.
    Per token and head, with ``q`` normalised and scaled by ``K**-0.5``:

        S <- Diag(exp(g_t)) S                 (gdn2.py:165)
        r  = S^T (b_t * k_t)                  (gdn2.py:168-169)
        u  = w_t * v_t - r                    (gdn2.py:172)
        S <- S + k_t u^T                      (gdn2.py:175)
        o_t = S^T q_t                         (gdn2.py:178)

    Returns ``(o [B,T,HV,V], final_state [N,HV,K,V])`` in float64; with
    ``return_states`` also the list of per-token states per sequence.
    """
    B, T, H, K = np.shape(q)
    HV, V = np.shape(v)[2], np.shape(v)[3]
    q, k, v, g, b, w = _prep(q, k, v, g, b, w, scale, use_qk_l2norm_in_kernel)
    q = _expand_heads(q, HV)
    k = _expand_heads(k, HV)
    seqs = _seq_slices(B, T, cu_seqlens)
    N = len(seqs)
    o = np.zeros((B, T, HV, V))
    final = np.zeros((N, HV, K, V))
    states = []
    for n, (bi, t0, t1) in enumerate(seqs):
        S = np.zeros((HV, K, V)) if initial_state is None else np.array(initial_state[n], dtype=np.float64)
        seq_states = []
        for t in range(t0, t1):
            S = S * np.exp(g[bi, t])[:, :, None]
            r = np.einsum("hkv,hk->hv", S, b[bi, t] * k[bi, t])
            u = w[bi, t] * v[bi, t] - r
            S = S + k[bi, t][:, :, None] * u[:, None, :]
            o[bi, t] = np.einsum("hkv,hk->hv", S, q[bi, t])
            if return_states:
                seq_states.append(S.copy())
        final[n] = S
        states.append(seq_states)
    if return_states:
        return o, final, states
    return o, final


def chunk_fwd(
    q,
    k,
    v,
    g,
    b,
    w,
    initial_state=None,
    scale=None,
    use_qk_l2norm_in_kernel=True,
    chunk_size=64,
):
    r"""Chunkwise (WY/UT) gdn2 forward in float64 with relative decays only.

    For one chunk with start state ``S0`` and in-chunk cumulative log decay
    ``G_r = sum_{i<=r} g_i`` (per key channel), with ``e_r = b_r * k_r`` and
    ``z_r = w_r * v_r``:

        Aqk[r,i] = sum_d q_rd k_id exp(G_rd - G_id)      i <= r
        L[r,i]   = sum_d e_rd k_id exp(G_rd - G_id)      i <  r
        X  = (I + L)^{-1}
        W  = X (e * exp(G)),   U0 = X z,   U = U0 - W S0
        O  = (q * exp(G)) S0 + Aqk U
        S1 = Diag(exp(G_last)) S0 + (k * exp(G_last - G))^T U

    This is the algebra of the HIP chunk kernels; it is checked against
    ``recurrent_fwd`` (the reference recurrence) for every chunk size.
    """
    B, T, H, K = np.shape(q)
    V = np.shape(v)[-1]
    q, k, v, g, b, w = _prep(q, k, v, g, b, w, scale, use_qk_l2norm_in_kernel)
    o = np.zeros((B, T, H, V))
    final = np.zeros((B, H, K, V))
    for bi in range(B):
        for h in range(H):
            S = np.zeros((K, V)) if initial_state is None else np.array(initial_state[bi, h], dtype=np.float64)
            for t0 in range(0, T, chunk_size):
                t1 = min(T, t0 + chunk_size)
                qc, kc, vc = q[bi, t0:t1, h], k[bi, t0:t1, h], v[bi, t0:t1, h]
                gc, bc, wc = g[bi, t0:t1, h], b[bi, t0:t1, h], w[bi, t0:t1, h]
                C = t1 - t0
                G = np.cumsum(gc, axis=0)  # [C,K]
                causal = np.tril(np.ones((C, C)))
                expo = np.where(causal[:, :, None] > 0, G[:, None, :] - G[None, :, :], -np.inf)
                rel = np.exp(expo)  # [C,C,K] indexed (r, i, d); zero above the diagonal
                strict = np.tril(np.ones((C, C)), -1)
                e = bc * kc
                Aqk = np.einsum("rd,id,rid->ri", qc, kc, rel) * causal
                L = np.einsum("rd,id,rid->ri", e, kc, rel) * strict
                X = np.linalg.inv(np.eye(C) + L)
                Wm = X @ (e * np.exp(G))
                U = X @ (wc * vc) - Wm @ S
                o[bi, t0:t1, h] = (qc * np.exp(G)) @ S + Aqk @ U
                S = np.exp(G[-1])[:, None] * S + (kc * np.exp(G[-1][None, :] - G)).T @ U
            final[bi, h] = S
    return o, final


def recurrent_fwd_pooled(
    q,
    k,
    v,
    g,
    b,
    w,
    state_pool,
    ssm_state_indices,
    num_accepted_tokens=None,
    inplace_final_state=True,
    scale=None,
    use_qk_l2norm_in_kernel=True,
    cu_seqlens=None,
    transpose_state_layout=False,
    final_rows=None,
):
    r"""Token-serial forward over a state pool (continuous batching).

    Restates the addressing of the reference kernel
    (``fused_recurrent_gdn2.py:215-232`` and ``:311-326``). The index entry of
    sequence ``n`` at position ``t`` is ``idx.flat[n * stride + t]``, where
    ``stride`` is 1 for ``[N]`` indices and ``T_max`` for ``[N, T_max]``.

    * **Initial state.** Sequence ``n`` starts from pool row ``idx[n, i0]``, with
      ``i0 = num_accepted_tokens[n] - 1`` if given, else 0.
    * **Per-token stores.** After each token ``t``, the state is stored to pool
      row ``idx[n, t]`` when ``inplace_final_state``. Otherwise it goes to row
      ``bos + t`` of a new array of ``final_rows`` rows.
    * **Padded entries.** An entry outside the index array, or a slot outside the
      pool, reads a zero state and stores nothing. The reference leaves that case
      unguarded; this is the HIP op's documented behaviour.
    * **Transposed layout.** With ``transpose_state_layout``, pool rows are
      ``[HV, V, K]``.
    * **Order.** All initial states are read before any store, so sequences must
      not share slots, as on the GPU.

    Returns ``(o, final, written)``:
    * ``final`` is the updated pool (in place) or the new array;
    * ``written`` is the sorted list of rows that were stored.
    """
    B, T = np.shape(q)[:2]
    HV, V, K = np.shape(v)[2], np.shape(v)[3], np.shape(q)[3]
    idx = np.asarray(ssm_state_indices)
    stride = 1 if idx.ndim == 1 else idx.shape[1]
    flat = idx.reshape(-1).astype(np.int64)
    pool = np.array(state_pool, dtype=np.float64)
    rows = pool.shape[0]
    seqs = _seq_slices(B, T, cu_seqlens)

    def slot(pos, nrows):
        if pos < 0 or pos >= flat.size:
            return -1
        s_ = int(flat[pos])
        return s_ if 0 <= s_ < nrows else -1

    def to_kv(x):
        return np.swapaxes(x, -1, -2) if transpose_state_layout else x

    if inplace_final_state:
        final = pool.copy()
    else:
        final = np.zeros((final_rows if final_rows is not None else len(seqs),) + pool.shape[1:])
    o = np.zeros((B, T, HV, V))
    written = set()
    pending = []
    for n, (bi, t0, t1) in enumerate(seqs):
        if t1 == t0:
            continue
        i0 = int(num_accepted_tokens[n]) - 1 if num_accepted_tokens is not None else 0
        s0 = slot(n * stride + i0, rows)
        h0 = np.zeros((1, HV, K, V)) if s0 < 0 else to_kv(pool[s0])[None]
        sl = (slice(bi, bi + 1), slice(t0, t1))
        on, _, states = recurrent_fwd(q[sl], k[sl], v[sl], g[sl], b[sl], w[sl], h0, scale=scale,
                                      use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                      return_states=True)
        o[bi, t0:t1] = on[0]
        for t, S in enumerate(states[0]):
            tok = bi * T + t0 + t  # packed token position (bos + t)
            row = slot(n * stride + t, final.shape[0]) if inplace_final_state else (
                tok if tok < final.shape[0] else -1)
            if row >= 0:
                pending.append((row, to_kv(S)))
    for row, S in pending:
        final[row] = S
        written.add(row)
    return o, final, sorted(written)


def short_conv(x, weight, bias=None, cache=None, output_final_state=False, activation="silu"):
    r"""Causal depthwise conv1d of ``x [B, T, D]`` in float64 (gdn2.py:395-430).

    ``weight`` is ``[D, W]`` (or the Conv1d ``[D, 1, W]``), ``bias`` ``[D]``.  Output
    ``y[b, t, d] = bias[d] + sum_j weight[d, j] * xp[b, t + j, d]`` with ``xp`` the
    inputs preceded by ``W-1`` tokens of history: the cache ``[B, D, W-1]`` on a
    single-token call with a cache (gdn2.py:409-412), zeros otherwise
    (padding=W-1, truncated to T, gdn2.py:414-424).  SiLU follows when
    ``activation == "silu"``.  The new cache (with ``output_final_state``) is the
    last ``W-1`` entries of the history + inputs on a single-token call, else
    the last ``min(T, W-1)`` inputs, as ``[B, D, n]``.
    """
    x = np.asarray(x, dtype=np.float64)
    B, T, D = x.shape
    w = np.asarray(weight, dtype=np.float64).reshape(D, -1)
    W = w.shape[1]
    if cache is not None and T == 1:
        hist = np.transpose(np.asarray(cache, dtype=np.float64), (0, 2, 1))
    else:
        hist = np.zeros((B, W - 1, D))
    xp = np.concatenate([hist, x], axis=1)
    y = np.zeros((B, T, D))
    for j in range(W):
        y += w[:, j] * xp[:, j:j + T, :]
    if bias is not None:
        y += np.asarray(bias, dtype=np.float64)
    if activation == "silu":
        y = y / (1.0 + np.exp(-y))
    new = None
    if output_final_state:
        if T == 1:
            new = np.transpose(xp[:, -(W - 1):, :], (0, 2, 1)) if W > 1 else np.zeros((B, D, 0))
        else:
            keep = min(T, W - 1)
            new = np.transpose(x[:, T - keep:, :], (0, 2, 1))
    return y, new


def gated_rmsnorm(x, z, weight, eps=1e-5):
    r"""``x * rsqrt(mean(x^2) + eps) * weight * silu(z)`` over the last axis, float64
    (gdn2.py:433-452)."""
    x = np.asarray(x, dtype=np.float64)
    z = np.asarray(z, dtype=np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return x * inv * np.asarray(weight, dtype=np.float64) * (z / (1.0 + np.exp(-z)))


def rmsnorm(x, weight, eps=1e-5):
    r"""``weight * x * rsqrt(mean(x^2) + eps)`` over the last axis, float64
    (models/normalization.py:40-51): the gated norm without its gate."""
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return x * inv * np.asarray(weight, dtype=np.float64)


def _l2norm_vjp(x_raw, dy, eps=L2_EPS):
    """VJP of ``y = x / max(||x||, eps)`` over the last axis."""
    n = np.sqrt((x_raw * x_raw).sum(-1, keepdims=True))
    big = n > eps
    nn = np.maximum(n, eps)
    y = x_raw / nn
    proj = (y * dy).sum(-1, keepdims=True)
    return np.where(big, (dy - y * proj) / nn, dy / eps)


def recurrent_vjp(
    q,
    k,
    v,
    g,
    b,
    w,
    do,
    dht=None,
    initial_state=None,
    scale=None,
    use_qk_l2norm_in_kernel=True,
):
    r"""Reverse-mode derivative of ``recurrent_fwd`` (no varlen, H == HV).

    Given the upstream gradients ``do [B,T,H,V]`` and optionally ``dht``
    ``[B,H,K,V]`` (gradient of the final state), returns
    ``(dq, dk, dv, dg, db, dw, dh0)`` with respect to the raw (un-normalised)
    inputs -- the set of gradients ``ChunkGDN2Function.backward`` returns
    (reference ``chunk_gdn2.py:2526-2547``).

    Per step, walking t = T-1 .. 0 with ``dS`` the gradient of ``S_t``:

        dS += q_t do_t^T ;  dq_t = S_t do_t
        dk_t = dS u_t ;  du = dS^T k_t
        dw_t = du * v_t ;  dv_t = du * w_t ;  dr = -du
        dS~ = dS + e_t dr^T ;  de = S~ dr
        db_t = de * k_t ;  dk_t += de * b_t
        dg_t = rowsum(dS~ * S~) ;  dS <- Diag(exp(g_t)) dS~
    """
    B, T, H, K = np.shape(q)
    V = np.shape(v)[-1]
    q_raw = np.asarray(q, dtype=np.float64)
    k_raw = np.asarray(k, dtype=np.float64)
    if scale is None:
        scale = K ** -0.5
    qs, kn, v, g, b, w = _prep(q, k, v, g, b, w, scale, use_qk_l2norm_in_kernel)
    do = np.asarray(do, dtype=np.float64)
    dq = np.zeros_like(qs)
    dk = np.zeros_like(kn)
    dv = np.zeros_like(v)
    dg = np.zeros_like(g)
    db = np.zeros_like(b)
    dw = np.zeros_like(w)
    dh0 = np.zeros((B, H, K, V))
    for bi in range(B):
        for h in range(H):
            S = np.zeros((K, V)) if initial_state is None else np.array(initial_state[bi, h], dtype=np.float64)
            Sdec, Ss, us = [], [], []
            for t in range(T):
                St = np.exp(g[bi, t, h])[:, None] * S
                e = b[bi, t, h] * kn[bi, t, h]
                u = w[bi, t, h] * v[bi, t, h] - St.T @ e
                S = St + np.outer(kn[bi, t, h], u)
                Sdec.append(St)
                Ss.append(S)
                us.append(u)
            dS = np.zeros((K, V)) if dht is None else np.array(dht[bi, h], dtype=np.float64)
            for t in range(T - 1, -1, -1):
                qt, kt, et = qs[bi, t, h], kn[bi, t, h], b[bi, t, h] * kn[bi, t, h]
                dS = dS + np.outer(qt, do[bi, t, h])
                dq[bi, t, h] = Ss[t] @ do[bi, t, h]
                dk_t = dS @ us[t]
                du = dS.T @ kt
                dw[bi, t, h] = du * v[bi, t, h]
                dv[bi, t, h] = du * w[bi, t, h]
                dr = -du
                dSt = dS + np.outer(et, dr)
                de = Sdec[t] @ dr
                db[bi, t, h] = de * kt
                dk_t = dk_t + de * b[bi, t, h]
                dk[bi, t, h] = dk_t
                dg[bi, t, h] = (dSt * Sdec[t]).sum(-1)
                dS = np.exp(g[bi, t, h])[:, None] * dSt
            dh0[bi, h] = dS
    dq = dq * scale
    if use_qk_l2norm_in_kernel:
        dq = _l2norm_vjp(q_raw, dq)
        dk = _l2norm_vjp(k_raw, dk)
    return dq, dk, dv, dg, db, dw, dh0


def chunk_vjp(
    q,
    k,
    v,
    g,
    b,
    w,
    do,
    dht=None,
    initial_state=None,
    scale=None,
    use_qk_l2norm_in_kernel=True,
    chunk_size=64,
):
    r"""Chunkwise reverse-mode derivative of ``chunk_fwd`` (no varlen, H == HV).

    Returns ``(dq, dk, dv, dg, db, dw, dh0)`` like ``recurrent_vjp``.  For one
    chunk (notation of ``chunk_fwd``; ``Qb = q*exp(G)``, ``Eb = e*exp(G)``,
    ``Kt = k*exp(G_last - G)``) with ``dS1`` the gradient of its end state:

        dU  = Aqk^T dO + Kt dS1,      dY = X^T dU     (dz = dY: dv = dY*w, dw = dY*v)
        dQb = dO S0^T,  dEb = -dY S0^T,  dKt = U dS1^T
        dA  = tril(dO U^T),  dL = strict_tril(-dY U^T)
        dq_r = exp(G_r) dQb_r + sum_j dA[r,j] k_j exp(G_r - G_j)
        de_r = exp(G_r) dEb_r + sum_j dL[r,j] k_j exp(G_r - G_j)
        dk_j = exp(G_last - G_j) dKt_j + sum_r (dA[r,j] q_r + dL[r,j] e_r) exp(G_r - G_j)
        dG_r = q_r dq_r + e_r de_r - k_r dk_r,   dG_last += rowsum(dS1 * S1)
        dg   = reverse in-chunk cumulative sum of dG
        dS0  = Qb^T dO + Diag(exp(G_last)) dS1 - Eb^T dY

    ``rowsum(dS1 * S1)`` is the whole derivative of ``S1`` with respect to
    ``G_last`` at fixed ``U`` (``S1 = exp(G_last) (S0 + sum_j exp(-G_j) k_j u_j^T)``).
    """
    B, T, H, K = np.shape(q)
    V = np.shape(v)[-1]
    q_raw = np.asarray(q, dtype=np.float64)
    k_raw = np.asarray(k, dtype=np.float64)
    if scale is None:
        scale = K ** -0.5
    qs, kn, v, g, b, w = _prep(q, k, v, g, b, w, scale, use_qk_l2norm_in_kernel)
    do = np.asarray(do, dtype=np.float64)
    dq, dk, dv = np.zeros_like(qs), np.zeros_like(kn), np.zeros_like(v)
    dg, db, dw = np.zeros_like(g), np.zeros_like(b), np.zeros_like(w)
    dh0 = np.zeros((B, H, K, V))
    for bi in range(B):
        for h in range(H):
            S = np.zeros((K, V)) if initial_state is None else np.array(initial_state[bi, h], dtype=np.float64)
            bounds = [(t0, min(T, t0 + chunk_size)) for t0 in range(0, T, chunk_size)]
            saved = []
            for t0, t1 in bounds:
                qc, kc = qs[bi, t0:t1, h], kn[bi, t0:t1, h]
                ec = b[bi, t0:t1, h] * kc
                zc = w[bi, t0:t1, h] * v[bi, t0:t1, h]
                G = np.cumsum(g[bi, t0:t1, h], axis=0)
                C = t1 - t0
                causal = np.tril(np.ones((C, C)))
                expo = np.where(causal[:, :, None] > 0, G[:, None, :] - G[None, :, :], -np.inf)
                rel = np.exp(expo)
                Aqk = np.einsum("rd,id,rid->ri", qc, kc, rel)
                L = np.einsum("rd,id,rid->ri", ec, kc, rel) * np.tril(np.ones((C, C)), -1)
                X = np.linalg.inv(np.eye(C) + L)
                Eb = ec * np.exp(G)
                Kt = kc * np.exp(G[-1][None, :] - G)
                U = X @ (zc - Eb @ S)
                saved.append((qc, kc, ec, G, rel, Aqk, X, Eb, Kt, S, U))
                S = np.exp(G[-1])[:, None] * S + Kt.T @ U
            ends = [saved[i + 1][9] for i in range(len(saved) - 1)] + [S]
            dS = np.zeros((K, V)) if dht is None else np.array(dht[bi, h], dtype=np.float64)
            for ci in range(len(bounds) - 1, -1, -1):
                t0, t1 = bounds[ci]
                qc, kc, ec, G, rel, Aqk, X, Eb, Kt, S0, U = saved[ci]
                dO = do[bi, t0:t1, h]
                dU = Aqk.T @ dO + Kt @ dS
                dY = X.T @ dU
                dv[bi, t0:t1, h] = dY * w[bi, t0:t1, h]
                dw[bi, t0:t1, h] = dY * v[bi, t0:t1, h]
                dA = np.tril(dO @ U.T)
                dL = np.tril(-dY @ U.T, -1)
                eG = np.exp(G)
                dqc = eG * (dO @ S0.T) + np.einsum("ri,id,rid->rd", dA, kc, rel)
                de = eG * (-dY @ S0.T) + np.einsum("ri,id,rid->rd", dL, kc, rel)
                dkc = (np.exp(G[-1][None, :] - G) * (U @ dS.T)
                       + np.einsum("ri,rd,rid->id", dA, qc, rel)
                       + np.einsum("ri,rd,rid->id", dL, ec, rel))
                dG = qc * dqc + ec * de - kc * dkc
                last = (dS * ends[ci]).sum(-1)
                dg[bi, t0:t1, h] = np.cumsum(dG[::-1], axis=0)[::-1] + last
                db[bi, t0:t1, h] = de * kc
                dk[bi, t0:t1, h] = dkc + de * b[bi, t0:t1, h]
                dq[bi, t0:t1, h] = dqc
                dS = (qc * eG).T @ dO + np.exp(G[-1])[:, None] * dS - Eb.T @ dY
            dh0[bi, h] = dS
    dq = dq * scale
    if use_qk_l2norm_in_kernel:
        dq = _l2norm_vjp(q_raw, dq)
        dk = _l2norm_vjp(k_raw, dk)
    return dq, dk, dv, dg, db, dw, dh0


def make_inputs(cfg_index: int, B, T, H, K, V, seed=None, scalar_gates=True, state_std=0.0):
    r"""Seeded synthetic inputs of the BASELINE configs (numpy float64).

    Draw order (a fixed contract): q, k, v, beta_logit, g_pre, then the
    initial state when ``state_std > 0``.  q and k ~ N(0,1) then L2-normalised
    per head; v ~ N(0,1); beta = sigmoid(N(0,1)); g = -softplus(N(0,1) + 2).
    With ``scalar_gates`` beta and g are drawn per (b, t, h) and broadcast to
    the channel-wise API (``g, b`` over K and ``w`` over V, with b = w = beta).
    """
    rng = np.random.default_rng(cfg_index if seed is None else seed)
    q = l2normalize(rng.standard_normal((B, T, H, K)))
    k = l2normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, H, V))
    gshape = (B, T, H, 1) if scalar_gates else (B, T, H, K)
    bl = rng.standard_normal(gshape)
    gp = rng.standard_normal(gshape)
    beta = 1.0 / (1.0 + np.exp(-bl))
    g = -np.logaddexp(0.0, gp + 2.0)
    if scalar_gates:
        g = np.broadcast_to(g, (B, T, H, K)).copy()
        bk = np.broadcast_to(beta, (B, T, H, K)).copy()
        wv = np.broadcast_to(beta, (B, T, H, V)).copy()
    else:
        bk = beta
        wv = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H, V))))
    h0 = None
    if state_std > 0:
        h0 = rng.standard_normal((B, H, K, V)) * state_std
    return dict(q=q, k=k, v=v, g=g, b=bk, w=wv, h0=h0)
